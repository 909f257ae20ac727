// common.hpp — shared helpers of the gfx950 kernel library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace nnhip
{

// Op codes shared with nn::ComputeEngine (compute_engine.hpp:43-82).
enum : unsigned { U_NEG = 0, U_EXP = 1, U_LOG = 2, U_SQRT = 3, U_RSQRT = 4, U_ABS = 5, U_TANH = 6 };
enum : unsigned { B_ADD = 0, B_SUB = 1, B_MUL = 2, B_DIV = 3, B_MAX = 4, B_MIN = 5 };
enum : unsigned { C_LT = 0, C_LE = 1, C_GT = 2, C_GE = 3, C_EQ = 4, C_NE = 5 };
enum : unsigned { R_SUM = 0, R_MAX = 1, R_MIN = 2 };

constexpr float kLowest = -3.40282347e+38f;   // std::numeric_limits<float>::lowest()
constexpr float kMaxF = 3.40282347e+38f;

// std::max / std::min semantics (first operand wins on ties and NaN in b).
__device__ __forceinline__ float fmax_std(float a, float b) { return (a < b) ? b : a; }
__device__ __forceinline__ float fmin_std(float a, float b) { return (b < a) ? b : a; }

__device__ __forceinline__ float unary_op(unsigned op, float x)
{
    switch (op)
    {
    case U_NEG: return -x;
    case U_EXP: return expf(x);
    case U_LOG: return logf(x);
    case U_SQRT: return sqrtf(x);
    case U_RSQRT: return 1.0f / sqrtf(x);
    case U_ABS: return fabsf(x);
    case U_TANH: return tanhf(x);
    default: return 0.0f;
    }
}

__device__ __forceinline__ float binary_op(unsigned op, float a, float b)
{
    switch (op)
    {
    case B_ADD: return a + b;
    case B_SUB: return a - b;
    case B_MUL: return a * b;
    case B_DIV: return a / b;
    case B_MAX: return fmax_std(a, b);
    case B_MIN: return fmin_std(a, b);
    default: return 0.0f;
    }
}

__device__ __forceinline__ bool compare_op(unsigned op, float a, float b)
{
    switch (op)
    {
    case C_LT: return a < b;
    case C_LE: return a <= b;
    case C_GT: return a > b;
    case C_GE: return a >= b;
    case C_EQ: return a == b;
    case C_NE: return a != b;
    default: return false;
    }
}

// Float-encoded row index as static_cast<size_t>(f) would read it: values in
// (-1, 2^64) truncate toward zero; valid iff the result is < rows.
__device__ __forceinline__ bool row_index(float f, size_t rows, size_t& out)
{
    if (!(f > -1.0f) || !(f < 1.8446744e19f)) return false;
    const size_t r = static_cast<size_t>(f);
    if (r >= rows) return false;
    out = r;
    return true;
}

__device__ __forceinline__ float wave_sum(float v)
{
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v)
{
    for (int o = 32; o > 0; o >>= 1) v = fmax_std(v, __shfl_xor(v, o, 64));
    return v;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline unsigned grid_for(size_t work, unsigned per_block, unsigned cap = 1u << 20)
{
    size_t g = (work + per_block - 1) / per_block;
    if (g == 0) g = 1;
    if (g > cap) g = cap;
    return static_cast<unsigned>(g);
}

// Launch status of the last kernel on this thread, as a C-ABI return code.
// CUs of the current device (cached per device; 256 when the query fails).
inline int device_cus()
{
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0)
    {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

inline int launch_status()
{
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : static_cast<int>(e);
}

} // namespace nnhip
