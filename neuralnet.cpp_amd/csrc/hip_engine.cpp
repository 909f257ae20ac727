// hip_engine.cpp — HipEngine: ComputeEngine primitives over the gfx950 kernel library.
//
// Each method mirrors the CPU engine's validation (cpu_engine.hpp, lines cited
// per method) and then enqueues the matching nnhip_* kernel on the engine's
// stream. The primitive semantics live in the kernels (include/nnhip_kernels.h).
#include "nn/hip_engine.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <limits>
#include <map>
#include <mutex>
#include <vector>

#include "nn/expr_dsl.hpp"
#include "nn/layer_exprs.hpp"
#include "nnhip_kernels.h"

namespace nn
{

// ── stream-ordered caching pool ────────────────────────────────────────────
// Blocks are rounded to size classes (powers of two up to 64 MiB, then 16 MiB
// multiples) and recycled by exact class. Every user of a pool enqueues on the
// same stream, so a block returned here may be handed out again right away:
// the kernels that read the old contents run before the ones that write it.
class DevicePool
{
public:
    explicit DevicePool(int device) : device_(device) {}
    ~DevicePool() { trim(); }

    static std::size_t round(std::size_t bytes)
    {
        if (bytes <= 256) return 256;
        constexpr std::size_t big = std::size_t{64} << 20, step = std::size_t{16} << 20;
        if (bytes >= big) return (bytes + step - 1) / step * step;
        std::size_t p = 256;
        while (p < bytes) p <<= 1;
        return p;
    }

    void* alloc(std::size_t bytes, std::size_t& rounded)
    {
        rounded = round(bytes);
        {
            std::lock_guard<std::mutex> lk(mu_);
            auto it = free_.find(rounded);
            if (it != free_.end() && !it->second.empty())
            {
                void* p = it->second.back();
                it->second.pop_back();
                cached_ -= rounded;
                live_ += rounded;
                return p;
            }
        }
        void* p = nullptr;
        (void)hipSetDevice(device_);
        if (hipMalloc(&p, rounded) != hipSuccess)
        {
            (void)hipGetLastError();
            (void)hipDeviceSynchronize();
            trim();
            if (hipMalloc(&p, rounded) != hipSuccess)
            {
                (void)hipGetLastError();
                return nullptr;
            }
        }
        std::lock_guard<std::mutex> lk(mu_);
        live_ += rounded;
        return p;
    }

    void release(void* p, std::size_t rounded)
    {
        std::lock_guard<std::mutex> lk(mu_);
        free_[rounded].push_back(p);
        live_ -= rounded;
        cached_ += rounded;
    }

    void trim()
    {
        std::lock_guard<std::mutex> lk(mu_);
        for (auto& [sz, v] : free_)
            for (void* p : v) (void)hipFree(p);
        free_.clear();
        cached_ = 0;
    }

    std::size_t cached() const
    {
        std::lock_guard<std::mutex> lk(mu_);
        return cached_;
    }
    std::size_t live() const
    {
        std::lock_guard<std::mutex> lk(mu_);
        return live_;
    }

private:
    int device_;
    mutable std::mutex mu_;
    std::map<std::size_t, std::vector<void*>> free_;
    std::size_t cached_ = 0, live_ = 0;
};

namespace
{

class HipBuffer final : public DeviceBuffer
{
public:
    HipBuffer(std::shared_ptr<DevicePool> pool, float* p, std::size_t floats, std::size_t rounded)
        : pool_(std::move(pool)), p_(p), floats_(floats), rounded_(rounded)
    {
    }
    ~HipBuffer() override
    {
        if (p_) pool_->release(p_, rounded_);
    }
    float* data() noexcept override { return p_; }
    std::size_t capacity() const noexcept override { return floats_; }

private:
    std::shared_ptr<DevicePool> pool_;
    float* p_;
    std::size_t floats_, rounded_;
};

// A row slice viewing rows of a root buffer (a pool block, or a view that
// holds a private copy). materialise() gives it its own block holding the
// same floats and drops the root; after that it is a root itself.
class HipView final : public DeviceBuffer
{
public:
    HipView(std::shared_ptr<DeviceBuffer> root, std::size_t offset, std::size_t floats)
        : root_(std::move(root)), off_(offset), floats_(floats)
    {
    }
    float* data() noexcept override { return own_ ? own_->data() : root_->data() + off_; }
    std::size_t capacity() const noexcept override { return floats_; }
    bool aliased() const noexcept { return !own_; }
    const DeviceBuffer* root() const noexcept { return root_.get(); }
    const std::shared_ptr<DeviceBuffer>& root_ptr() const noexcept { return root_; }
    std::size_t offset() const noexcept { return off_; }
    void materialise(std::shared_ptr<DeviceBuffer> own)
    {
        own_ = std::move(own);
        root_.reset();
    }

private:
    std::shared_ptr<DeviceBuffer> root_, own_;
    std::size_t off_, floats_;
};

const float* D(const Tensor& t) { return t.dev_ptr(); }
float* W(const Tensor& t) { return t.dev_ptr(); }

struct BDims
{
    std::size_t M, K, N;
};
Result<BDims> bdims(const Tensor& A, const Tensor& B, std::size_t batch, bool tA, bool tB, const char* who)
{
    if (batch == 0) return fail(std::string(who) + ": batch must be > 0");
    if (A.rows() % batch != 0 || B.rows() % batch != 0) return fail(std::string(who) + ": rows not divisible by batch");
    const std::size_t ar = A.rows() / batch, br = B.rows() / batch;
    BDims d{tA ? A.cols() : ar, tA ? ar : A.cols(), tB ? br : B.cols()};
    if (d.K != (tB ? B.cols() : br)) return fail(std::string(who) + ": K dimension mismatch");
    return d;
}
Result<void> mask_ok(const Tensor* mask, std::size_t M, std::size_t N, const char* who)
{
    if (mask && (mask->rows() != M || mask->cols() != N)) return fail(std::string(who) + ": mask shape mismatch");
    return {};
}
Result<void> vec_ok(const Tensor& t, std::size_t rows, const char* who, const char* what)
{
    if (t.rows() != rows || t.cols() != 1) return fail(std::string(who) + ": " + what + " shape mismatch");
    return {};
}

// A layer program (include/nn/layer_exprs.hpp) in canonical form, with the
// argument each input slot of the folded spec reads.
struct Canon
{
    ExprSpec spec;
    std::vector<int> arg_of_slot;
    int nargs = 0;
};

template <class Build>
Canon make_canon(int nargs, Build build)
{
    std::vector<Tensor> a;
    for (int i = 0; i < nargs; ++i) a.push_back(Tensor::cpu(static_cast<std::size_t>(i) + 1, 1));
    auto [spec, ins] = dsl::to_expr_spec(build(a));
    Canon c{std::move(spec), {}, nargs};
    for (const Tensor& t : ins) c.arg_of_slot.push_back(static_cast<int>(t.rows()) - 1);
    return c;
}

// True when `spec` is the canonical program and all slots of one argument
// hold the same device tensor; args[] then receives one pointer per argument.
bool bind(const Canon& c, const ExprSpec& spec, std::span<const Tensor> inputs, const float** args)
{
    if (inputs.size() != c.arg_of_slot.size() || !expr_spec_equal(spec, c.spec)) return false;
    for (int i = 0; i < c.nargs; ++i) args[i] = nullptr;
    for (std::size_t k = 0; k < inputs.size(); ++k)
    {
        const float*& a = args[c.arg_of_slot[k]];
        const float* p = inputs[k].dev_ptr();
        if (a == nullptr)
            a = p;
        else if (a != p)
            return false;
    }
    return true;
}

enum class LayerProg
{
    SoftmaxFwd, SoftmaxBwd, RmsSumSq, RmsNormalize, RmsScale, RmsBwdColSum, RmsBwdDx, RmsBwdRowSum, SwigluGate,
    SwigluUp, Count
};

const Canon& canon(LayerProg p)
{
    namespace le = layer_exprs;
    static const Canon table[] = {
        make_canon(1, [](auto& a) { return le::softmax_rows(a[0]); }),
        make_canon(2, [](auto& a) { return le::softmax_rows_backward(a[0], a[1]); }),
        make_canon(1, [](auto& a) { return le::rms_sum_sq(a[0]); }),
        make_canon(2, [](auto& a) { return le::rms_normalize(a[0], a[1]); }),
        make_canon(2, [](auto& a) { return le::rms_scale(a[0], a[1]); }),
        make_canon(3, [](auto& a) { return le::rms_bwd_colsum(a[0], a[1], a[2]); }),
        make_canon(5, [](auto& a) { return le::rms_bwd_dx(a[0], a[1], a[2], a[3], a[4]); }),
        make_canon(3, [](auto& a) { return le::rms_bwd_rowsum(a[0], a[1], a[2]); }),
        make_canon(4, [](auto& a) { return le::swiglu_grad_gate(a[0], a[1], a[2], a[3]); }),
        make_canon(3, [](auto& a) { return le::swiglu_grad_up(a[0], a[1], a[2]); }),
    };
    static_assert(sizeof table / sizeof table[0] == static_cast<std::size_t>(LayerProg::Count));
    return table[static_cast<int>(p)];
}

// ── deferred attention chains ───────────────────────────────────────────────
bool same_t(const Tensor& a, const Tensor& b)
{
    return a.dev_ptr() && a.dev_ptr() == b.dev_ptr() && a.rows() == b.rows() && a.cols() == b.cols();
}
bool same_mask(const Tensor* a, const std::optional<Tensor>& b) { return a ? (b && same_t(*a, *b)) : !b; }
bool has_buf(const Tensor& t, const float* p) { return p && t.dev_ptr() == p; }
bool in_buf(const Tensor& t, const float* p)
{
    const float* b = t.dev_ptr();
    return p && b && p >= b && p < b + (t.size() ? t.size() : 1);
}
bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }
// True when a tensor held by a deferred record is also referenced elsewhere.
bool live(const Tensor& t) { return t.device_buffer().use_count() > 1; }

} // namespace

// reduce(Max) [-> softmax_denom]: m (and l) still to be computed.
struct HipEngine::PendingFwd
{
    Tensor Q, K;
    std::optional<Tensor> mask;
    std::size_t batch, M, N, Kd;
    float alpha;
    Tensor m;
    std::optional<Tensor> l;
    bool uses(const float* p) const
    {
        return has_buf(Q, p) || has_buf(K, p) || (mask && has_buf(*mask, p)) || has_buf(m, p) ||
               (l && has_buf(*l, p));
    }
    bool yields(const float* p) const { return has_buf(m, p) || (l && has_buf(*l, p)); }
    bool matches(const Tensor& A, const Tensor& B, std::size_t b, bool tA, bool tB, Scalar a, const Tensor* mk) const
    {
        return same_t(A, Q) && same_t(B, K) && b == batch && tA && !tB && a == alpha && same_mask(mk, mask);
    }
};

// batched_matmul(A, B, transA, !transB): its product C still to be computed.
struct HipEngine::PendingGemm
{
    Tensor A, B, C;
    std::size_t batch, M, N, K;
    float alpha;
    bool uses(const float* p) const { return has_buf(A, p) || has_buf(B, p) || has_buf(C, p); }
    bool yields(const float* p) const { return has_buf(C, p); }
};

// softmax_backward_q on a deferred product P: dQ and R still to be computed.
struct HipEngine::PendingBwd
{
    Tensor Q, K, P, m, l;
    std::optional<Tensor> mask;
    std::size_t batch, M, N, Kd;
    float alpha;
    Tensor dQ, R;
    bool uses(const float* p) const
    {
        return has_buf(Q, p) || has_buf(K, p) || has_buf(P, p) || has_buf(m, p) || has_buf(l, p) ||
               (mask && has_buf(*mask, p)) || has_buf(dQ, p) || has_buf(R, p);
    }
    bool yields(const float* p) const { return has_buf(dQ, p) || has_buf(R, p); }
};

enum EwCode : std::uint8_t { kBin, kScalar, kUnary, kAxpy, kCopy };

// One call of a recognised chain of deferred elementwise calls: code, op,
// scalar-first flag and the roles of its destination and operands (b < 0: not read).
struct RunStep
{
    EwCode code;
    unsigned op;
    std::uint8_t first;
    int dst, a, b;
};

// A SwiGLU gradient program (SwiGLU::backward) not launched yet. The layer
// inserts each result into its (2 d_ff, N) gradient right away; the program
// then writes those rows directly (`placed`), both programs in one pass when
// both are placed.
struct HipEngine::PendingSwb
{
    bool up;                      // grad_up (G, gate, s) or grad_gate (G, up, s, gate)
    Tensor G, upt, s, gate, out;  // upt: unused by grad_up
    Tensor dst;
    std::size_t off = 0;          // floats into dst
    bool placed = false;
    bool uses(const float* p) const
    {
        return has_buf(G, p) || has_buf(upt, p) || has_buf(s, p) || has_buf(gate, p) || has_buf(out, p) ||
               (placed && has_buf(dst, p));
    }
};

// matmul(A, B) not launched yet (see HipEngine::matmul). `folded`: its product
// was already added into another tensor; C itself is computed only if read.
struct HipEngine::PendingMm
{
    Tensor A, B, C;
    bool tA, tB;
    std::size_t M, N, K;
    bool folded;
    Tensor bias;   // the Linear bias added by the call that followed (broadcast_row_inplace), if any
    Tensor heads;  // C already written in the heads' layout (B_h sequences of N_h) by a grouped launch
    std::size_t heads_B = 0, heads_N = 0;
    // Further products A^T B of the same shape added into C (add_inplace(C, their outputs)): C is their
    // sum, computed as one product over the concatenated K (transposed A only).
    std::vector<std::pair<Tensor, Tensor>> plus;
    // A matrix-vector product's second destination: out2 (from element out2_off) = addx + C (the block's
    // residual add) or, without addx, a copy of C (insert_rows of C's transpose into a KV cache).
    Tensor out2, addx;
    std::size_t out2_off = 0;
    bool uses(const float* p) const
    {
        for (const auto& [a, b] : plus)
            if (has_buf(a, p) || has_buf(b, p)) return true;
        return has_buf(A, p) || has_buf(B, p) || in_buf(C, p) || has_buf(bias, p) || has_buf(out2, p) ||
               has_buf(addx, p);
    }
    // Anywhere in C: a row slice of a recorded matrix-vector product (slice_rows
    // leaves it recorded) is read through a pointer into it.
    bool yields(const float* p) const { return in_buf(C, p) || has_buf(out2, p); }
    bool needed() const { return live(C) || (out2.size() && live(out2)); }
};

// Weight-gradient accumulations C_i += A_i op(B_i) (Linear::backward's
// grad_w += G X^T, folded into the product) of one shape, not launched yet:
// the attention's output, q, k and v layers have d_model x d_model weights
// (q, k and v share their input X), so their four accumulations run as one
// grouped launch (nnhip_gemm_group_acc[_each]).
struct HipEngine::PendingAcc
{
    Tensor B;   // member 0's
    bool tB;
    std::size_t M, N, K;
    std::vector<std::pair<Tensor, Tensor>> mem;   // (A_i, C_i)
    std::vector<Tensor> mb;                       // B_i
    bool acc = true;                              // C_i += A_i op(B), else C_i = A_i op(B)
    // Linear::backward's grad_b += row_reduce_sum(G) of a member (A_i = G): the
    // row sums go to rs[i] (added when rs_acc), computed by the same launch.
    std::vector<Tensor> rs;
    int rs_acc = -1;
    bool yields(const float* p) const
    {
        for (const auto& m : mem)
            if (has_buf(m.second, p)) return true;
        for (const auto& t : rs)
            if (has_buf(t, p)) return true;
        return false;
    }
    bool uses(const float* p) const
    {
        for (const auto& m : mem)
            if (has_buf(m.first, p)) return true;
        for (const auto& t : mb)
            if (has_buf(t, p)) return true;
        return yields(p) || has_buf(B, p);
    }
};

// Consecutive same-size elementwise calls (scale / axpy / add in place; unary,
// binary, scalar and clone into new tensors), recorded in call order. Slots
// are the distinct buffers the calls touch; every result is a real allocation
// that the record keeps alive until it runs.
struct HipEngine::PendingEw
{
    struct Op
    {
        EwCode code;
        std::uint8_t op, first;
        std::uint8_t dst, a, b;   // slots; b is read by kBin and kAxpy only
        float s;
    };
    static constexpr std::size_t kMaxOps = 96, kMaxSlots = 64;
    std::size_t n = 0;   // elements of every tensor in the record
    std::vector<Tensor> slots;
    std::vector<Op> ops;
    // Some slots are row slices of a recorded matrix-vector product that was
    // left unlaunched (SwiGLU's gate and up halves of a token's fc1): the
    // product runs before the record, or with it (swiglu_vec_run_).
    bool vec_reads = false;

    std::uint8_t slot(const Tensor& t)
    {
        for (std::size_t i = 0; i < slots.size(); ++i)
            if (slots[i].dev_ptr() == t.dev_ptr()) return static_cast<std::uint8_t>(i);
        slots.push_back(t);
        return static_cast<std::uint8_t>(slots.size() - 1);
    }
    bool full() const { return ops.size() >= kMaxOps || slots.size() + 3 > kMaxSlots; }
    static bool reads_b(const Op& o) { return o.code == kBin || o.code == kAxpy; }
};

// The reference's materialised attention (compute_layer.hpp:1230-1252 forward,
// :1331-1361 backward), recorded call by call and run by the one-pass kernels:
//   scores = batched_matmul(Q, K, transA) * alpha      PendingGemm
//   masked = scores + mask                             PendingMaskAdd
//   A      = softmax rows of masked                    PendingAttn (kept per layer)
//   O      = batched_matmul(V, A, transB)              fused forward: O, and m, l into the record
//   dV     = batched_matmul(dO, A)                     PendingDv
//   P      = batched_matmul(dO, V, transA)             PendingGemm
//   dS     = softmax backward (A, P)                   PendingDs
//   dQ     = batched_matmul(K, dS, transB) * alpha     fused backward: dQ, dK, dV (AttnGrads)
//   dK     = batched_matmul(Q, dS) * alpha
// Each record can also compute its result with the general kernels, which is
// what happens when anything else reads it or writes one of its inputs.
struct HipEngine::PendingMaskAdd
{
    Tensor Q, K, mask, out;   // out = alpha * Q^T K (per batch) + mask
    std::size_t batch, M, N, Kd;
    float alpha;
    bool uses(const float* p) const
    {
        return has_buf(Q, p) || has_buf(K, p) || has_buf(mask, p) || has_buf(out, p);
    }
};
struct HipEngine::PendingAttn
{
    Tensor Q, K, mask, A;     // A: the probabilities handed out; written only when materialised
    std::size_t batch, M, N, Kd;
    float alpha;
    Tensor m, l;              // row max and sum, once the fused forward has run
    Tensor V, O;              // the fused forward's values and output (R_i = dO_i . O_i in the backward)
    bool stats = false, materialised = false;
    bool scores = false;      // A's memory holds the fused forward's score blocks (until materialised)
    bool uses(const float* p) const
    {
        return has_buf(Q, p) || has_buf(K, p) || has_buf(mask, p) || has_buf(A, p) || has_buf(V, p) ||
               has_buf(O, p);
    }
};
struct HipEngine::PendingDv
{
    std::shared_ptr<PendingAttn> p;
    Tensor dO, out;           // out = dO A (per batch)
    bool uses(const float* q) const { return has_buf(dO, q) || has_buf(out, q) || p->uses(q); }
};
struct HipEngine::PendingDs
{
    std::shared_ptr<PendingAttn> p;
    Tensor dO, Vp, out;       // out = A * (P - rowsum(A P)), P = alpha2 * dO^T Vp (per batch)
    std::size_t Kd2;
    float alpha2;
    bool uses(const float* q) const
    {
        return has_buf(dO, q) || has_buf(Vp, q) || has_buf(out, q) || p->uses(q);
    }
};
// dQ and dK of a fused backward, waiting for their batched_matmul calls.
struct HipEngine::AttnGrads
{
    Tensor dS, Q, K, dQ, dK;
    float alpha;
    bool q_taken = false, k_taken = false;
};

// transpose(S) not launched yet, or the per-batch transpose that
// rearrange_3d(transpose(S), M, B, N) makes of it: out rows [b*M, (b+1)*M)
// are the transpose of S rows [b*N, (b+1)*N). The two-pass attention turns V
// and dO from per batch (d_k, seq) into (seq, d_k) this way
// (compute_layer.hpp:1211-1214, :1309-1313); its kernels read S in place
// instead, and anything else that reads out gets the copy.
struct HipEngine::PendingLayout
{
    Tensor S, out;
    bool per_batch;
    std::size_t M, B, N;   // per_batch: out (B*M, N) from S (B*N, M)
    // merge: out (M, B*N) = rearrange_3d(S, M, B, N, inverse), S (B*M, N)
    // holding the heads' rows (the attention's per-sequence layout)
    bool merge = false;
    bool uses(const float* p) const { return has_buf(S, p) || has_buf(out, p); }
};

// row_reduce_sum(src), or RMSNorm::backward's row sums of src * gamma[r] *
// normed (kind 1), not launched yet: the layer's next call adds them into its
// gradient (Linear::backward's grad_b += row_reduce_sum(G), RMSNorm's
// grad_gamma += gg), which the row-sum kernel then does itself; `out` is
// computed only if it is read later (`folded`: the sums were already added).
struct HipEngine::PendingRowSum
{
    Tensor src, out, gamma, normed;
    int kind = 0;
    bool folded = false;
    bool uses(const float* p) const
    {
        return has_buf(src, p) || has_buf(out, p) || has_buf(gamma, p) || has_buf(normed, p);
    }
};

// RMSNorm::forward (compute_layer.hpp RMSNorm) as the layer issues it:
//   s       = eval_expr_reduce(sum of squares, x)       stage 1
//   scaled  = s * inv_f                                 stage 2
//   var_eps = scaled + eps                              stage 3
//   rinv    = rsqrt(var_eps)                            stage 4
//   normed  = eval_expr(normalize, x, rinv)             stage 5
//   out     = eval_expr(scale, normed, gamma)           one nnhip_rmsnorm_forward pass
// and RMSNorm::backward's first three calls (bwd):
//   m_raw   = eval_expr_reduce(g gamma normed, column sums)   stage 1 (x = g, s = m_raw)
//   m       = m_raw * inv_f                                    stage 2 (scaled = m)
//   dx      = eval_expr(dx program, g, gamma, m, normed, rinv) one nnhip_rmsnorm_backward pass
// Each call returns its tensor unlaunched; any other use of one of them (or a
// write to an input) runs the calls so far with their separate kernels.
struct HipEngine::PendingRms
{
    bool bwd = false;
    Tensor x, s, scaled, var_eps, rinv, normed;
    Tensor gamma;   // bwd: with x = g and normed, an input; forward stage 6: the scale
    Tensor y;       // forward stage 6 (one column): the output, normed * gamma
    // forward: x = xa + xb, a recorded elementwise_binary(Add) taken into the
    // launch (GPTBlock::forward's residual add before the layer); x is an output
    Tensor xa, xb;
    Tensor dx;      // bwd stage 3: dx, not launched yet (rinv is then an input)
    float inv_f = 0.0f, eps = 0.0f;
    int stage = 1;
    bool yields(const float* p) const
    {
        if (bwd) return has_buf(s, p) || has_buf(scaled, p) || has_buf(dx, p);
        return has_buf(s, p) || has_buf(scaled, p) || has_buf(var_eps, p) || has_buf(rinv, p) || has_buf(normed, p) ||
               has_buf(y, p) || (xa.size() && has_buf(x, p));
    }
    bool uses(const float* p) const
    {
        return has_buf(x, p) || yields(p) || has_buf(gamma, p) || (bwd && (has_buf(normed, p) || has_buf(rinv, p))) ||
               has_buf(xa, p) || has_buf(xb, p);
    }
};

// The two-pass chain's softmax_apply output O (per batch (M, D), query-major)
// with what it came from; V was read from Vs (per batch (D, N)). The backward
// takes R_i = alpha2 dO_i . O_i from it instead of a second score pass.
struct HipEngine::TwoPassOut
{
    Tensor Q, K;
    std::optional<Tensor> mask;
    Tensor m, l, Vs, O;
    std::size_t batch;
    float alpha;
    Tensor S;   // the forward's score blocks for the backward, or empty
    bool uses(const float* p) const
    {
        return has_buf(Q, p) || has_buf(K, p) || (mask && has_buf(*mask, p)) || has_buf(m, p) || has_buf(l, p) ||
               has_buf(Vs, p) || has_buf(O, p);
    }
};

// A fused two-pass launch not run yet: the forward of softmax_apply (m, l, O
// and the score blocks S from Q, K and V read dim-major from Vs) or the
// backward of backward_kv from that forward's output (R, dQ, dK, dV from Q,
// K, dO, V' = Vs, O, m, l and S). The cell table is held so that its address
// stays this mask's while the record waits.
struct HipEngine::PendingFlash
{
    bool bwd = false;
    Tensor Q, K, Vs, dO, O, m, l, S, R, dQ, dK, dV;
    std::optional<Tensor> mask;
    std::shared_ptr<DeviceBuffer> cells;
    std::size_t batch = 0, M = 0, N = 0, Kd = 0, D = 0;
    float alpha = 0.0f, alpha2 = 0.0f;
    bool v_dm = false;   // forward: Vs per batch (D, N) (the recorded layout's source) instead of (N, D)
    bool yields(const float* p) const
    {
        if (bwd) return has_buf(R, p) || has_buf(dQ, p) || has_buf(dK, p) || has_buf(dV, p);
        return has_buf(O, p) || has_buf(m, p) || has_buf(l, p) || has_buf(S, p);
    }
    bool uses(const float* p) const
    {
        return yields(p) || has_buf(Q, p) || has_buf(K, p) || has_buf(Vs, p) || has_buf(dO, p) ||
               (mask && has_buf(*mask, p)) || (bwd && (has_buf(O, p) || has_buf(m, p) || has_buf(l, p) ||
                                                       has_buf(S, p)));
    }
    // Records that run as rows of one launch.
    bool joins(const PendingFlash& o) const
    {
        return bwd == o.bwd && batch == o.batch && M == o.M && N == o.N && Kd == o.Kd && D == o.D &&
               !mask == !o.mask && !S.size() == !o.S.size() && alpha == o.alpha && alpha2 == o.alpha2 &&
               v_dm == o.v_dm;
    }
};

namespace
{

// The Adam update chain of one parameter tensor as the optimizer issues it
// (reference compute_optimizer.hpp:252-304): the tensors it touches, by role,
// and its calls in order. AdamW (:388-412) puts scale_inplace(p, decay) first.
enum AdamRole { rP, rM, rG, rV, rG2, rMH, rVH, rSQ, rDEN, rR, kAdamRoles };
constexpr unsigned kMul = static_cast<unsigned>(BinaryOp::Mul), kAdd = static_cast<unsigned>(BinaryOp::Add),
                   kDiv = static_cast<unsigned>(BinaryOp::Div), kSqrt = static_cast<unsigned>(UnaryOp::Sqrt),
                   kNeg = static_cast<unsigned>(UnaryOp::Neg), kExp = static_cast<unsigned>(UnaryOp::Exp);
constexpr RunStep kAdamSteps[] = {
    {kScalar, kMul, 0, rP, rP, -1},       // p *= 1 - lr * wd (AdamW only)
    {kScalar, kMul, 0, rM, rM, -1},       // m *= beta1
    {kAxpy, 0, 0, rM, rM, rG},            // m += (1 - beta1) g
    {kScalar, kMul, 0, rV, rV, -1},       // v *= beta2
    {kBin, kMul, 0, rG2, rG, rG},         // g2 = g * g
    {kScalar, kMul, 0, rG2, rG2, -1},     // g2 *= 1 - beta2
    {kBin, kAdd, 0, rV, rV, rG2},         // v += g2
    {kCopy, 0, 0, rMH, rM, -1},           // m_hat = clone(m)
    {kScalar, kMul, 0, rMH, rMH, -1},     // m_hat *= inv_bc1
    {kCopy, 0, 0, rVH, rV, -1},           // v_hat = clone(v)
    {kScalar, kMul, 0, rVH, rVH, -1},     // v_hat *= inv_bc2
    {kUnary, kSqrt, 0, rSQ, rVH, -1},     // sq = sqrt(v_hat)
    {kScalar, kAdd, 0, rDEN, rSQ, -1},    // den = sq + eps
    {kBin, kDiv, 0, rR, rMH, rDEN},       // ratio = m_hat / den
    {kScalar, kMul, 0, rR, rR, -1},       // ratio *= -lr
    {kBin, kAdd, 0, rP, rP, rR},          // p += ratio
};
constexpr std::size_t kAdamLen = sizeof(kAdamSteps) / sizeof(kAdamSteps[0]) - 1;   // without the decay

// SwiGLU::forward's chain (its sigmoid written out as primitives).
enum SwigluRole { sG, sU, sT1, sT2, sT3, sS, sSW, sO, kSwigluRoles };
constexpr RunStep kSwigluSteps[] = {
    {kUnary, kNeg, 0, sT1, sG, -1},       // t1 = -gate
    {kUnary, kExp, 0, sT2, sT1, -1},      // t2 = exp(t1)
    {kScalar, kAdd, 0, sT3, sT2, -1},     // t3 = t2 + 1
    {kScalar, kDiv, 1, sS, sT3, -1},      // s = 1 / t3
    {kBin, kMul, 0, sSW, sG, sS},         // sw = gate * s
    {kBin, kMul, 0, sO, sSW, sU},         // out = sw * up
};
constexpr std::size_t kSwigluLen = sizeof(kSwigluSteps) / sizeof(kSwigluSteps[0]);

} // namespace

HipEngine::HipEngine()
{
    if (hipGetDevice(&device_) != hipSuccess)
    {
        init_error_ = "HipEngine: no HIP device";
        (void)hipGetLastError();
        return;
    }
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess)
    {
        init_error_ = "HipEngine: hipStreamCreate failed";
        (void)hipGetLastError();
        return;
    }
    stream_ = s;
    pool_ = std::make_shared<DevicePool>(device_);
    // Score blocks kept from forward to backward: at most 1/8 of the memory
    // free now and at most 8 GiB.
    std::size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess)
    {
        (void)hipGetLastError();
        free_b = 0;
    }
    score_budget_ = std::min(std::size_t(8) << 30, free_b / 8);
    ok_ = true;
}

HipEngine::~HipEngine()
{
    if (stream_)
    {
        (void)hipStreamSynchronize(static_cast<hipStream_t>(stream_));
        (void)hipStreamDestroy(static_cast<hipStream_t>(stream_));
    }
    for (auto& r : prof_)
    {
        (void)hipEventDestroy(static_cast<hipEvent_t>(r.start));
        (void)hipEventDestroy(static_cast<hipEvent_t>(r.stop));
    }
    for (void* e : event_pool_) (void)hipEventDestroy(static_cast<hipEvent_t>(e));
    for (void* e : stage_ev_)
        if (e) (void)hipEventDestroy(static_cast<hipEvent_t>(e));
    if (stage_) (void)hipHostFree(stage_);
}

// ── GEMM event profile ──────────────────────────────────────────────────────
// Turning the profile on creates the events of the launches to come first
// (two per GEMM; 8192 cover a default bench run of 10 config-4 steps), so the
// profiled region records events without creating them.
void HipEngine::set_gemm_profile(bool on)
{
    profile_ = on;
    constexpr std::size_t kReserve = 8192;
    while (on && event_pool_.size() < kReserve)
    {
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess)
        {
            (void)hipGetLastError();
            break;
        }
        event_pool_.push_back(e);
    }
}

void HipEngine::prof_begin_()
{
    if (!profile_) return;
    auto take = [this]() -> void* {
        if (!event_pool_.empty())
        {
            void* e = event_pool_.back();
            event_pool_.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        (void)hipEventCreate(&e);
        return e;
    };
    ProfRecord r{take(), take(), 0.0, {}};
    (void)hipEventRecord(static_cast<hipEvent_t>(r.start), static_cast<hipStream_t>(stream_));
    prof_.push_back(r);
}

void HipEngine::prof_end_(std::size_t M, std::size_t N, std::size_t K, std::size_t batch, bool tA, bool tB)
{
    if (!profile_ || prof_.empty()) return;
    ProfRecord& r = prof_.back();
    r.flops = 2.0 * double(batch) * double(M) * double(N) * double(K);
    const double shape[6] = {double(M), double(N), double(K), double(batch), tA ? 1.0 : 0.0, tB ? 1.0 : 0.0};
    std::copy(shape, shape + 6, r.shape);
    (void)hipEventRecord(static_cast<hipEvent_t>(r.stop), static_cast<hipStream_t>(stream_));
}

Result<void> HipEngine::read_gemm_profile(double& launches, double& flops, double& ms)
{
    std::vector<double> rec;
    NN_CHECK(read_gemm_profile_records(rec));
    launches = static_cast<double>(rec.size() / 7);
    flops = 0.0;
    ms = 0.0;
    for (std::size_t i = 0; i + 7 <= rec.size(); i += 7)
    {
        flops += 2.0 * rec[i] * rec[i + 1] * rec[i + 2] * rec[i + 3];
        ms += rec[i + 6];
    }
    return {};
}

Result<void> HipEngine::read_gemm_profile_records(std::vector<double>& records)
{
    NN_CHECK(end_batch());
    records.clear();
    for (auto& r : prof_)
    {
        float t = 0.0f;
        if (hipEventElapsedTime(&t, static_cast<hipEvent_t>(r.start), static_cast<hipEvent_t>(r.stop)) != hipSuccess)
            return fail("read_gemm_profile: event timing failed");
        records.insert(records.end(), r.shape, r.shape + 6);
        records.push_back(t);
        event_pool_.push_back(r.start);
        event_pool_.push_back(r.stop);
    }
    prof_.clear();
    return {};
}

std::size_t HipEngine::pool_cached_bytes() const { return pool_ ? pool_->cached() : 0; }
std::size_t HipEngine::pool_live_bytes() const { return pool_ ? pool_->live() : 0; }

Result<void> HipEngine::kernel_(int rc, const char* what)
{
    if (rc == 0) return {};
    if (rc > 0)
        return fail(std::string(what) + ": HIP error " + hipGetErrorString(static_cast<hipError_t>(rc)));
    if (rc == -3) return fail(std::string(what) + ": shape outside this kernel's supported range");
    return fail(std::string(what) + ": invalid arguments (status " + std::to_string(rc) + ")");
}

Result<void> HipEngine::check_gpu_(std::initializer_list<const Tensor*> ts, const char* what) const
{
    for (const Tensor* t : ts)
        if (t && (!t->is_gpu() || (t->size() > 0 && !t->dev_ptr())))
            return fail(std::string(what) + ": tensor is not on this GPU engine");
    return {};
}

Result<void> HipEngine::need_gpu_(std::initializer_list<const Tensor*> ts, const char* what)
{
    NN_CHECK(check_gpu_(ts, what));
    return settle_reads_(ts);
}

// ── deferred work: launch on demand ─────────────────────────────────────────
Result<void> HipEngine::settle_reads_(std::initializer_list<const Tensor*> ts)
{
    NN_CHECK(settle_ew_());
    return settle_chain_reads_(ts);
}

Result<void> HipEngine::settle_chain_reads_(std::initializer_list<const Tensor*> ts, bool keep_flash)
{
    for (const Tensor* t : ts)
    {
        if (!t) continue;
        const float* p = t->dev_ptr();
        if (!p) continue;
        NN_CHECK(settle_zero_for_(*t));
        if (pacc_ && pacc_->yields(p)) NN_CHECK(settle_acc_());
        if (!keep_flash && flash_yields_(p)) NN_CHECK(settle_flash_());
        if (pmm_ && pmm_->yields(p)) NN_CHECK(settle_mm_());
        if (!pmm_prev_.empty()) NN_CHECK(settle_mm_prev_(p, false));
        for (const auto& r : pswb_)
            if (has_buf(r.out, p) || (r.placed && has_buf(r.dst, p)))
            {
                NN_CHECK(settle_swb_());
                break;
            }
        if (pmadd_ && has_buf(pmadd_->out, p)) NN_CHECK(settle_madd_());
        if (prms_ && prms_->yields(p)) NN_CHECK(settle_rms_());
        if (prsum_ && has_buf(prsum_->out, p)) NN_CHECK(settle_rsum_());
        for (std::size_t i = 0; i < playout_.size(); ++i)
            if (has_buf(playout_[i].out, p))
            {
                const PendingLayout r = std::move(playout_[i]);
                playout_.erase(playout_.begin() + static_cast<std::ptrdiff_t>(i));
                NN_CHECK(materialise_layout_(r));
                break;
            }
        if (pdv_ && has_buf(pdv_->out, p)) NN_CHECK(settle_dv_());
        if (pds_ && has_buf(pds_->out, p)) NN_CHECK(settle_ds_());
        for (auto& a : pattn_)
            if (has_buf(a->A, p)) NN_CHECK(materialise_attn_(*a));
        if (pbwd_ && pbwd_->yields(p)) NN_CHECK(settle_bwd_());
        if (pgemm_ && pgemm_->yields(p)) NN_CHECK(settle_gemm_());
        if (pfwd_ && pfwd_->yields(p)) NN_CHECK(settle_fwd_());
    }
    return {};
}

// Cell tables of a mask tensor read as rows / M stacked (M, N) masks (one
// table each), cached per tensor until it is written in place or evicted.
Result<std::shared_ptr<DeviceBuffer>> HipEngine::mask_cells_buf_(const Tensor* mask, std::size_t M, std::size_t N)
{
    if (!mask) return std::shared_ptr<DeviceBuffer>();
    for (std::size_t i = 0; i < cells_.size(); ++i)
        if (same_t(cells_[i].mask, *mask) && cells_[i].M == M)
        {
            CellTable t = cells_[i];
            cells_.erase(cells_.begin() + static_cast<std::ptrdiff_t>(i));
            cells_.push_back(t);
            return t.cells;
        }
    const std::size_t masks = mask->rows() / M;
    NN_TRY(buf, scratch_(masks * nnhip_flash_cells_bytes(M, N)));
    NN_CHECK(kernel_(nnhip_flash_classify_batched(D(*mask), masks, M * N, M, N, buf->data(), stream_),
                     "attention mask cells"));
    constexpr std::size_t kKeep = 32;   // one per layer's mask in a 12-32 layer model
    if (cells_.size() == kKeep) cells_.erase(cells_.begin());
    cells_.push_back({*mask, buf, M, {}});
    return buf;
}

Result<const void*> HipEngine::mask_cells_(const Tensor* mask, std::size_t M, std::size_t N)
{
    NN_TRY(buf, mask_cells_buf_(mask, M, N));
    return static_cast<const void*>(buf ? buf->data() : nullptr);
}

// Work order of a multi-row launch (kind as flash_order_), built once per set
// of cell tables and shape; the last few are kept.
Result<const void*> HipEngine::rows_order_(const std::vector<std::shared_ptr<DeviceBuffer>>& cells, std::size_t hpr,
                                           std::size_t M, std::size_t N, int kind)
{
    for (std::size_t i = 0; i < rows_orders_.size(); ++i)
    {
        const RowsOrder& o = rows_orders_[i];
        if (o.cells == cells && o.hpr == hpr && o.M == M && o.N == N && o.kind == kind)
            return static_cast<const void*>(o.buf->data());
    }
    std::vector<const void*> ptrs;
    for (const auto& c : cells) ptrs.push_back(c->data());
    NN_TRY(buf, scratch_(nnhip_flash_order_bytes(cells.size() * hpr, M, N, kind)));
    NN_CHECK(kernel_(nnhip_flash_build_rows_order(ptrs.data(), cells.size(), hpr, M, N, kind, buf->data(), stream_),
                     "attention work order"));
    constexpr std::size_t kKeep = 8;
    if (rows_orders_.size() == kKeep) rows_orders_.erase(rows_orders_.begin());
    rows_orders_.push_back(RowsOrder{cells, hpr, M, N, kind, buf});
    return static_cast<const void*>(buf->data());
}

// ── recorded fused attention launches ───────────────────────────────────────
bool HipEngine::flash_yields_(const float* p) const
{
    for (const PendingFlash& r : pflash_)
        if (r.yields(p)) return true;
    return false;
}

bool HipEngine::flash_uses_(const float* p) const
{
    for (const PendingFlash& r : pflash_)
        if (r.uses(p)) return true;
    return false;
}

// Every recorded launch: the forwards, then the backwards (a backward reads
// only forwards' results; records of one kind never read each other's),
// records that join each other as rows of one launch, at most
// NNHIP_FLASH_MAX_ROWS per launch, in call order otherwise.
Result<void> HipEngine::settle_flash_()
{
    if (pflash_.empty()) return {};
    std::vector<PendingFlash> rs = std::move(pflash_);
    pflash_.clear();
    for (int kind = 0; kind < 2; ++kind)
    {
        std::vector<bool> done(rs.size(), false);
        for (std::size_t i = 0; i < rs.size(); ++i)
        {
            if (done[i] || rs[i].bwd != (kind == 1)) continue;
            std::vector<const PendingFlash*> rows{&rs[i]};
            done[i] = true;
            for (std::size_t j = i + 1; j < rs.size() && rows.size() < NNHIP_FLASH_MAX_ROWS; ++j)
                if (!done[j] && rs[j].joins(rs[i]))
                {
                    rows.push_back(&rs[j]);
                    done[j] = true;
                }
            NN_CHECK(launch_flash_(rows));
        }
    }
    return {};
}

Result<void> HipEngine::launch_flash_(const std::vector<const PendingFlash*>& rows)
{
    const PendingFlash& f = *rows.front();
    const std::size_t n = rows.size();
    std::vector<std::shared_ptr<DeviceBuffer>> cells;
    for (const PendingFlash* r : rows)
        if (r->cells) cells.push_back(r->cells);
    const void* order = nullptr;
    if (f.mask)
    {
        // One row: the table cached with its mask; several: one per set of tables.
        if (n == 1)
        {
            NN_TRY(o, flash_order_(f.cells->data(), f.batch, f.M, f.N, 0, f.bwd ? 2 : 0));
            order = o;
        }
        else
        {
            NN_TRY(o, rows_order_(cells, f.batch, f.M, f.N, f.bwd ? 2 : 0));
            order = o;
        }
    }
    if (!f.bwd)
    {
        std::vector<nnhip_flash_fwd_row> a(n);
        for (std::size_t r = 0; r < n; ++r)
        {
            const PendingFlash& x = *rows[r];
            a[r] = nnhip_flash_fwd_row{D(x.Q), D(x.K), D(x.Vs), x.mask ? D(*x.mask) : nullptr,
                                       x.cells ? x.cells->data() : nullptr, W(x.m), W(x.l), W(x.O),
                                       x.S.size() ? W(x.S) : nullptr};
        }
        NN_TRY(ws, scratch_(nnhip_flash_workspace_bytes(n * f.batch, f.M, f.N, f.Kd, f.D, 0)));
        return kernel_(nnhip_flash_forward_rows(a.data(), n, f.batch, f.M, f.N, f.Kd, f.D, f.alpha, f.v_dm ? 1 : 0,
                                                0, order, ws->data(), stream_),
                       "batched_matmul_softmax_apply");
    }
    std::vector<nnhip_flash_bwd_row> a(n);
    for (std::size_t r = 0; r < n; ++r)
    {
        const PendingFlash& x = *rows[r];
        a[r] = nnhip_flash_bwd_row{D(x.Q), D(x.K), D(x.dO), D(x.Vs), D(x.O), x.mask ? D(*x.mask) : nullptr,
                                   x.cells ? x.cells->data() : nullptr, D(x.m), D(x.l), x.S.size() ? D(x.S) : nullptr,
                                   W(x.R), W(x.dQ), W(x.dK), W(x.dV)};
    }
    NN_TRY(ws, scratch_(nnhip_flash_ds_workspace_bytes(n * f.batch, f.M, f.N, f.Kd)));
    return kernel_(nnhip_flash_backward_ds_rows(a.data(), n, f.batch, f.M, f.N, f.Kd, f.alpha, f.alpha2, 1, order,
                                                ws->data(), stream_),
                   "batched_matmul_softmax_backward_kv");
}

// Work order of a one-pass attention launch over a cached cell table (kind 0
// forward, 1 backward, 2 backward from the forward output), built once per
// table and shape and kept with the table.
Result<const void*> HipEngine::flash_order_(const void* cells, std::size_t batch, std::size_t M, std::size_t N,
                                            std::size_t mask_bs, int kind)
{
    // One query line per batch entry (a token of incremental inference, whose
    // mask is new every call): every entry visits the same cells, nothing to balance.
    if (!cells || M <= 32) return static_cast<const void*>(nullptr);
    for (CellTable& t : cells_)
    {
        if (t.cells->data() != cells) continue;
        const bool pb = mask_bs != 0;
        for (const OrderTable& o : t.orders)
            if (o.batch == batch && o.N == N && o.kind == kind && o.per_batch == pb)
                return static_cast<const void*>(o.buf->data());
        NN_TRY(buf, scratch_(nnhip_flash_order_bytes(batch, M, N, kind)));
        NN_CHECK(kernel_(nnhip_flash_build_order(cells, batch, M, N, mask_bs, kind, buf->data(), stream_),
                         "attention work order"));
        t.orders.push_back({batch, N, kind, pb, buf});
        return static_cast<const void*>(buf->data());
    }
    return static_cast<const void*>(nullptr);
}

Result<void> HipEngine::settle_write_(const Tensor& t)
{
    NN_CHECK(settle_ew_());
    return settle_chain_write_(t);
}

Result<void> HipEngine::settle_chain_write_(const Tensor& t, bool keep_swb, bool keep_zero)
{
    NN_CHECK(unshare_(t));
    const float* p = t.dev_ptr();
    if (!p) return {};
    if (!keep_zero) NN_CHECK(settle_zero_for_(t));
    if (pacc_ && pacc_->uses(p)) NN_CHECK(settle_acc_());
    if (flash_uses_(p)) NN_CHECK(settle_flash_());
    if (pmm_ && pmm_->uses(p)) NN_CHECK(settle_mm_());
    if (!pmm_prev_.empty()) NN_CHECK(settle_mm_prev_(p, true));
    for (const auto& r : pswb_)
        if (!keep_swb && r.uses(p))
        {
            NN_CHECK(settle_swb_());
            break;
        }
    if (pmadd_ && pmadd_->uses(p)) NN_CHECK(settle_madd_());
    if (prms_ && prms_->uses(p)) NN_CHECK(settle_rms_());
    if (prsum_ && prsum_->uses(p)) NN_CHECK(settle_rsum_());
    for (std::size_t i = playout_.size(); i-- > 0;)
    {
        if (i >= playout_.size()) continue;   // (a materialisation may settle others)
        if (playout_[i].uses(p))
        {
            const PendingLayout r = std::move(playout_[i]);
            playout_.erase(playout_.begin() + static_cast<std::ptrdiff_t>(i));
            if (live(r.out)) NN_CHECK(materialise_layout_(r));
        }
    }
    std::erase_if(ptwo_, [p](const TwoPassOut& r) { return r.uses(p); });
    if (pdv_ && pdv_->uses(p)) NN_CHECK(settle_dv_());
    if (pds_ && pds_->uses(p)) NN_CHECK(settle_ds_());
    if (pgrads_ && (has_buf(pgrads_->dQ, p) || has_buf(pgrads_->dK, p))) pgrads_.reset();
    for (std::size_t i = pattn_.size(); i-- > 0;)
        if (pattn_[i]->uses(p))
        {
            if (live(pattn_[i]->A)) NN_CHECK(materialise_attn_(*pattn_[i]));
            pattn_.erase(pattn_.begin() + static_cast<std::ptrdiff_t>(i));
        }
    for (std::size_t i = cells_.size(); i-- > 0;)
        if (has_buf(cells_[i].mask, p)) cells_.erase(cells_.begin() + static_cast<std::ptrdiff_t>(i));
    if (pbwd_ && pbwd_->uses(p)) NN_CHECK(settle_bwd_());
    if (pgemm_ && pgemm_->uses(p))
    {
        if (pbwd_ && same_t(pbwd_->P, pgemm_->C)) NN_CHECK(settle_bwd_());
        NN_CHECK(settle_gemm_());
    }
    if (pfwd_ && pfwd_->uses(p)) NN_CHECK(settle_fwd_());
    return {};
}

Result<void> HipEngine::settle_for_read(const Tensor& t)
{
    if (!t.is_gpu()) return {};
    return settle_reads_({&t});
}

Result<void> HipEngine::settle()
{
    NN_CHECK(settle_zero_());
    NN_CHECK(settle_ew_());
    NN_CHECK(settle_flash_());
    NN_CHECK(settle_acc_());
    NN_CHECK(settle_mm_());
    NN_CHECK(settle_mm_prev_(nullptr, false));
    NN_CHECK(settle_swb_());
    NN_CHECK(settle_madd_());
    NN_CHECK(settle_rms_());
    NN_CHECK(settle_rsum_());
    NN_CHECK(settle_dv_());
    NN_CHECK(settle_ds_());
    if (pgrads_ && !live(pgrads_->dQ) && !live(pgrads_->dK)) pgrads_.reset();
    forget_dead_attn_();
    forget_dead_two_();
    NN_CHECK(settle_bwd_());
    NN_CHECK(settle_gemm_());
    NN_CHECK(settle_fwd_());
    // Recorded transposes last: the records dropped above release the ones
    // only they referenced (the one-query attention's key and value operands).
    return settle_layout_();
}

// m (and l) of a deferred forward chain, in one pass over the scores.
Result<void> HipEngine::settle_fwd_()
{
    if (!pfwd_) return {};
    std::unique_ptr<PendingFwd> f = std::move(pfwd_);
    if (!live(f->m) && !(f->l && live(*f->l))) return {};
    Tensor l;
    if (f->l)
        l = *f->l;
    else
    {
        NN_TRY(t, alloc_(f->batch * f->M, 1));
        l = t;
    }
    NN_TRY(cells, mask_cells_(f->mask ? &*f->mask : nullptr, f->M, f->N));
    NN_TRY(order, flash_order_(cells, f->batch, f->M, f->N, 0, 0));
    NN_TRY(ws, scratch_(nnhip_flash_workspace_bytes(f->batch, f->M, f->N, f->Kd, 4, 0)));
    return kernel_(nnhip_flash_forward_ordered(D(f->Q), D(f->K), nullptr, f->mask ? D(*f->mask) : nullptr, cells,
                                               W(f->m), W(l), nullptr, f->batch, f->M, f->N, f->Kd, 4, f->alpha, 0, 0,
                                               0, nullptr, order, ws->data(), stream_),
                   "batched_matmul_reduce");
}

Result<void> HipEngine::settle_gemm_()
{
    if (!pgemm_) return {};
    if (pbwd_ && same_t(pbwd_->P, pgemm_->C)) NN_CHECK(settle_bwd_());
    if (!pgemm_) return {};
    std::unique_ptr<PendingGemm> g = std::move(pgemm_);
    if (!live(g->C)) return {};
    return launch_gemm_(g->A, g->B, g->C, g->batch, true, false, g->alpha, g->M, g->N, g->K);
}

// dQ and R of a deferred backward_q with the general kernels (P computed first).
Result<void> HipEngine::settle_bwd_()
{
    if (!pbwd_) return {};
    NN_CHECK(settle_flash_());   // m and l may come from a recorded forward
    if (!pbwd_) return {};
    std::unique_ptr<PendingBwd> q = std::move(pbwd_);
    if (!live(q->dQ) && !live(q->R)) return {};
    if (pgemm_ && same_t(q->P, pgemm_->C)) NN_CHECK(settle_gemm_());
    NN_TRY(ws, attn_ws_(q->batch, q->M, q->N, q->Kd, 1));
    return kernel_(nnhip_bmm_softmax_backward_q(D(q->Q), D(q->K), D(q->P), D(q->m), D(q->l),
                                                q->mask ? D(*q->mask) : nullptr, W(q->dQ), W(q->R), q->batch, q->M,
                                                q->N, q->Kd, 1, 0, q->alpha, ws ? ws->data() : nullptr, stream_),
                   "batched_matmul_softmax_backward_q");
}

// ── deferred materialised attention ─────────────────────────────────────────
void HipEngine::forget_dead_attn_()
{
    for (std::size_t i = pattn_.size(); i-- > 0;)
        if (!live(pattn_[i]->A) && pattn_[i].use_count() == 1) pattn_.erase(pattn_.begin() + static_cast<std::ptrdiff_t>(i));
}

void HipEngine::forget_dead_two_()
{
    std::erase_if(ptwo_, [](const TwoPassOut& r) { return !live(r.m) || !live(r.l); });
}

// ── recorded transposes ─────────────────────────────────────────────────────
Result<void> HipEngine::push_layout_(PendingLayout r)
{
    std::erase_if(playout_, [](const PendingLayout& q) { return !live(q.out); });
    // at most 16 transposes and 64 merges (the merges of a model's attention
    // layers are kept from the forward to the backward) recorded
    const std::size_t keep = r.merge ? 64 : 16;
    std::size_t n = 0;
    for (const PendingLayout& q : playout_) n += q.merge == r.merge;
    if (n >= keep)
        for (std::size_t i = 0; i < playout_.size(); ++i)
            if (playout_[i].merge == r.merge)
            {
                const PendingLayout o = std::move(playout_[i]);
                playout_.erase(playout_.begin() + static_cast<std::ptrdiff_t>(i));
                NN_CHECK(materialise_layout_(o));
                break;
            }
    playout_.push_back(std::move(r));
    return {};
}

Result<void> HipEngine::materialise_layout_(const PendingLayout& r)
{
    // (the source may be a recorded matrix-vector product, see transpose)
    if (const float* sp = r.S.dev_ptr(); sp)
    {
        if (pmm_ && pmm_->yields(sp)) NN_CHECK(settle_mm_());
        if (!pmm_prev_.empty()) NN_CHECK(settle_mm_prev_(sp, false));
    }
    if (r.merge)
    {
        NN_CHECK(settle_chain_reads_({&r.S}));
        return kernel_(nnhip_rearrange_3d(D(r.S), W(r.out), r.M, r.B, r.N, 1u, stream_), "rearrange_3d");
    }
    if (!r.per_batch)
        return kernel_(nnhip_transpose(D(r.S), W(r.out), r.S.rows(), r.S.cols(), stream_), "transpose");
    return kernel_(nnhip_transpose_batched(D(r.S), W(r.out), r.B, r.N, r.M, stream_), "rearrange_3d");
}

// Copies still referenced are made; the others are dropped. Merges stay
// recorded (read in place by the products that take them, made when anything
// else reads them or writes their rows).
Result<void> HipEngine::settle_layout_()
{
    std::vector<PendingLayout> rs = std::move(playout_);
    playout_.clear();
    for (PendingLayout& r : rs)
        if (r.merge && live(r.out)) playout_.push_back(std::move(r));
    for (const PendingLayout& r : rs)
        if (!r.merge && r.out.dev_ptr() && live(r.out)) NN_CHECK(materialise_layout_(r));
    return {};
}

const HipEngine::PendingLayout* HipEngine::layout_of_(const Tensor& t) const
{
    for (const PendingLayout& r : playout_)
        if (!r.merge && same_t(r.out, t)) return &r;
    return nullptr;
}

const HipEngine::PendingLayout* HipEngine::merge_of_(const Tensor& t) const
{
    for (const PendingLayout& r : playout_)
        if (r.merge && same_t(r.out, t)) return &r;
    return nullptr;
}

// The copy of a recorded transpose whose result t is about to be read (a
// no-op when t is not one).
Result<void> HipEngine::settle_layout_for_(const Tensor& t)
{
    for (std::size_t i = 0; i < playout_.size(); ++i)
        if (has_buf(playout_[i].out, t.dev_ptr()))
        {
            const PendingLayout r = std::move(playout_[i]);
            playout_.erase(playout_.begin() + static_cast<std::ptrdiff_t>(i));
            return materialise_layout_(r);
        }
    return {};
}

std::shared_ptr<HipEngine::PendingAttn> HipEngine::attn_of_(const Tensor& A) const
{
    for (const auto& a : pattn_)
        if (same_t(a->A, A)) return a;
    return nullptr;
}

// masked = alpha Q^T K + mask into `out` with the general kernels.
Result<void> HipEngine::scores_masked_(const Tensor& Q, const Tensor& K, const Tensor& mask, std::size_t batch,
                                       std::size_t M, std::size_t N, std::size_t Kd, float alpha, const Tensor& out)
{
    Tensor o = out;
    NN_CHECK(launch_gemm_(Q, K, o, batch, true, false, alpha, M, N, Kd));
    return kernel_(nnhip_elementwise_binary(D(out), D(mask), W(out), out.size(), 0u, stream_), "attention mask add");
}

Result<void> HipEngine::settle_madd_()
{
    if (!pmadd_) return {};
    std::unique_ptr<PendingMaskAdd> r = std::move(pmadd_);
    if (!live(r->out)) return {};
    return scores_masked_(r->Q, r->K, r->mask, r->batch, r->M, r->N, r->Kd, r->alpha, r->out);
}

// A = softmax rows (alpha Q^T K + mask), written into the handed-out tensor.
Result<void> HipEngine::materialise_attn_(PendingAttn& p)
{
    if (p.materialised) return {};
    NN_TRY(t, alloc_(p.batch * p.M, p.N));
    NN_CHECK(scores_masked_(p.Q, p.K, p.mask, p.batch, p.M, p.N, p.Kd, p.alpha, t));
    NN_CHECK(kernel_(nnhip_row_softmax(D(t), W(p.A), p.batch * p.M, p.N, stream_), "attention probabilities"));
    p.materialised = true;
    return {};
}

Result<void> HipEngine::settle_dv_()
{
    if (!pdv_) return {};
    std::unique_ptr<PendingDv> r = std::move(pdv_);
    if (!live(r->out)) return {};
    NN_CHECK(materialise_attn_(*r->p));
    const PendingAttn& p = *r->p;
    return launch_gemm_(r->dO, p.A, r->out, p.batch, false, false, 1.0f, r->dO.rows() / p.batch, p.N, p.M);
}

Result<void> HipEngine::settle_ds_()
{
    if (!pds_) return {};
    std::unique_ptr<PendingDs> r = std::move(pds_);
    if (!live(r->out)) return {};
    NN_CHECK(materialise_attn_(*r->p));
    const PendingAttn& p = *r->p;
    NN_TRY(P, alloc_(p.batch * p.M, p.N));
    NN_CHECK(launch_gemm_(r->dO, r->Vp, P, p.batch, true, false, r->alpha2, p.M, p.N, r->Kd2));
    return kernel_(nnhip_row_softmax_backward(D(p.A), D(P), W(r->out), p.batch * p.M, p.N, stream_),
                   "attention softmax backward");
}

// The calls of the chain that consume deferred tensors. Each returns nullopt
// when the call is not the expected next step; the caller then proceeds with
// the general path (which settles what it reads).
Result<std::optional<Tensor>> HipEngine::attn_bmm_(const Tensor& A, const Tensor& B, std::size_t batch, bool tA,
                                                   bool tB, Scalar alpha)
{
    using R = std::optional<Tensor>;
    // dQ / dK of a fused backward already run.
    if (pgrads_ && same_t(B, pgrads_->dS) && !tA && alpha == pgrads_->alpha)
    {
        if (tB && !pgrads_->q_taken && same_t(A, pgrads_->K))
        {
            pgrads_->q_taken = true;
            R r(pgrads_->dQ);
            if (pgrads_->k_taken) pgrads_.reset();
            return r;
        }
        if (!tB && !pgrads_->k_taken && same_t(A, pgrads_->Q))
        {
            pgrads_->k_taken = true;
            R r(pgrads_->dK);
            if (pgrads_->q_taken) pgrads_.reset();
            return r;
        }
    }
    if (tA) return R();
    auto p = attn_of_(B);
    // O = V A^T per batch: the fused forward.
    if (p && tB && !p->stats && alpha == 1.0f && A.rows() % batch == 0 && batch == p->batch && A.cols() == p->N)
    {
        const std::size_t Dv = A.rows() / batch;
        if (p->M == 1 && Dv > 0 && Dv <= 64 && p->Kd <= 64) return attn_query_(*p, A, Dv);
        if (Dv == 0 || !nnhip_flash_supported(batch, p->M, p->N, p->Kd, Dv)) return R();
        NN_CHECK(settle_reads_({&A}));
        NN_CHECK(settle_layout_for_(p->K));
        NN_TRY(out, alloc_(batch * Dv, p->M));
        NN_TRY(m, alloc_(batch * p->M, 1));
        NN_TRY(l, alloc_(batch * p->M, 1));
        NN_TRY(cells, mask_cells_(&p->mask, p->M, p->N));
        const std::size_t bs = p->mask.rows() == p->M ? 0 : p->M * p->N;
        NN_TRY(order, flash_order_(cells, batch, p->M, p->N, bs, 0));
        NN_TRY(ws, scratch_(nnhip_flash_workspace_bytes(batch, p->M, p->N, p->Kd, Dv, 0)));
        // The scores go to A's memory (the probabilities, written only if read through the engine),
        // one 32 x 32 block per cell, when M and N are whole tiles (then the blocks fill it exactly).
        const bool keep_scores = !p->materialised && p->M % 32 == 0 && p->N % 32 == 0;
        NN_CHECK(kernel_(nnhip_flash_forward_ordered(D(p->Q), D(p->K), D(A), D(p->mask), cells, W(m), W(l), W(out),
                                                     batch, p->M, p->N, p->Kd, Dv, p->alpha, bs, 1, 1,
                                                     keep_scores ? W(p->A) : nullptr, order, ws->data(), stream_),
                         "attention forward"));
        p->m = m;
        p->l = l;
        p->V = A;
        p->O = out;
        p->stats = true;
        p->scores = keep_scores;
        return R(out);
    }
    // dV = dO A per batch: recorded for the fused backward.
    if (p && !tB && p->stats && alpha == 1.0f && A.rows() == batch * p->Kd && A.cols() == p->M && batch == p->batch)
    {
        NN_CHECK(settle_reads_({&A}));
        NN_CHECK(settle_dv_());
        NN_TRY(out, alloc_(batch * p->Kd, p->N));
        pdv_ = std::make_unique<PendingDv>(PendingDv{p, A, out});
        return R(out);
    }
    // dQ = alpha K dS^T or dK = alpha Q dS per batch: run the fused backward.
    if (pds_ && same_t(B, pds_->out) && alpha == pds_->p->alpha &&
        ((tB && same_t(A, pds_->p->K)) || (!tB && same_t(A, pds_->p->Q))))
    {
        const PendingAttn& q = *pds_->p;
        NN_CHECK(settle_ew_());
        const bool dv_here = pdv_ && pdv_->p == pds_->p && same_t(pdv_->dO, pds_->dO);
        if (!dv_here) NN_CHECK(settle_dv_());
        NN_TRY(dQ, alloc_(batch * q.Kd, q.M));
        NN_TRY(dK, alloc_(batch * q.Kd, q.N));
        Tensor dV;
        if (dv_here)
            dV = pdv_->out;
        else
        {
            NN_TRY(t, alloc_(batch * q.Kd, q.N));
            dV = t;
        }
        NN_TRY(cells, mask_cells_(&q.mask, q.M, q.N));
        const std::size_t bs = q.mask.rows() == q.M ? 0 : q.M * q.N;
        NN_CHECK(settle_layout_for_(q.K));
        if (q.O.dev_ptr() && same_t(pds_->Vp, q.V) && q.V.rows() == batch * q.Kd)
        {
            // R from the forward output (same V): one key-line pass plus dQ from the stored dS.
            NN_TRY(order, flash_order_(cells, batch, q.M, q.N, bs, 2));
            NN_TRY(ws, scratch_(nnhip_flash_ds_workspace_bytes(batch, q.M, q.N, q.Kd)));
            NN_CHECK(kernel_(nnhip_flash_backward_ds_ordered(D(q.Q), D(q.K), D(pds_->dO), D(pds_->Vp), D(q.O), 0,
                                                             D(q.mask), cells, D(q.m), D(q.l), nullptr, W(dQ), W(dK),
                                                             W(dV), batch, q.M, q.N, q.Kd, q.alpha, pds_->alpha2, bs,
                                                             q.scores && !q.materialised ? D(q.A) : nullptr, order,
                                                             ws->data(), stream_),
                             "attention backward"));
        }
        else
        {
            NN_TRY(Rr, alloc_(batch * q.M, 1));
            NN_TRY(order, flash_order_(cells, batch, q.M, q.N, bs, 1));
            NN_TRY(ws, scratch_(nnhip_flash_workspace_bytes(batch, q.M, q.N, q.Kd, 4, 1)));
            NN_CHECK(kernel_(nnhip_flash_backward_ordered(D(q.Q), D(q.K), D(pds_->dO), D(pds_->Vp), nullptr, 0,
                                                          D(q.mask), cells, D(q.m), D(q.l), W(Rr), W(dQ), W(dK),
                                                          W(dV), batch, q.M, q.N, q.Kd, pds_->Kd2, q.alpha,
                                                          pds_->alpha2, bs, 1, order, ws->data(), stream_),
                             "attention backward"));
        }
        if (dv_here) pdv_.reset();
        pgrads_ = std::make_unique<AttnGrads>(AttnGrads{pds_->out, q.Q, q.K, dQ, dK, q.alpha});
        return attn_bmm_(A, B, batch, tA, tB, alpha);
    }
    return R();
}

// O = V A^T for one query per batch entry (incremental inference): m, l and O
// of the recorded chain in one launch, keys and values read where they lie
// (the KV cache rows when K and V are recorded transposes of them).
Result<std::optional<Tensor>> HipEngine::attn_query_(PendingAttn& p, const Tensor& V, std::size_t Dv)
{
    const std::size_t batch = p.batch, N = p.N, Kd = p.Kd;
    // Source rows of a recorded transpose: (N, batch * d) for a (batch * d, N) operand.
    auto rows_of = [&](const Tensor& t, std::size_t d) -> const Tensor* {
        const PendingLayout* l = layout_of_(t);
        return l && !l->per_batch && l->S.rows() == N && l->S.cols() == batch * d ? &l->S : nullptr;
    };
    const Tensor* ks = rows_of(p.K, Kd);
    const Tensor* vs = rows_of(V, Dv);
    if (ks) NN_CHECK(settle_chain_reads_({ks}));
    else NN_CHECK(settle_layout_for_(p.K));
    if (vs) NN_CHECK(settle_chain_reads_({vs}));
    else NN_CHECK(settle_reads_({&V}));
    const long kb = ks ? (long)Kd : (long)(Kd * N), kj = ks ? (long)ks->cols() : 1L, kk = ks ? 1L : (long)N;
    const long vb = vs ? (long)Dv : (long)(Dv * N), vj = vs ? (long)vs->cols() : 1L, vd = vs ? 1L : (long)N;
    const bool has_mask = p.mask.size() > 0;
    const long mask_bs = has_mask && p.mask.rows() != 1 ? static_cast<long>(N) : 0L;
    NN_TRY(out, alloc_(batch * Dv, 1));
    NN_TRY(m, alloc_(batch, 1));
    NN_TRY(l, alloc_(batch, 1));
    const std::size_t wsb = nnhip_attn_query_workspace_bytes(batch, N, Dv);
    std::shared_ptr<DeviceBuffer> ws;
    if (wsb)
    {
        NN_TRY(w, scratch_(wsb));
        ws = w;
    }
    // The probabilities go to the handed-out A as well (batch * N floats): the
    // record is then complete and dropped, and with it the key and value
    // operands, whose transposes are never made.
    NN_CHECK(kernel_(nnhip_attn_query(D(p.Q), ks ? D(*ks) : D(p.K), kb, kj, kk, vs ? D(*vs) : D(V), vb, vj, vd,
                                      has_mask ? D(p.mask) : nullptr, mask_bs, W(m), W(l), W(out), W(p.A), batch, N,
                                      Kd, Dv, p.alpha, ws ? ws->data() : nullptr, stream_),
                     "attention (one query)"));
    p.materialised = true;
    std::erase_if(pattn_, [&](const std::shared_ptr<PendingAttn>& q) { return q.get() == &p; });
    return std::optional<Tensor>(out);
}

// ── deferred elementwise runs ───────────────────────────────────────────────
// Records one call; a record of another size, or a full one, is launched first.
// The caller has checked shapes and launched deferred attention work that
// yields or reads the tensors involved.
Result<void> HipEngine::ew_push_(unsigned code, unsigned op, bool first, const Tensor& dst, const Tensor& a,
                                 const Tensor* b, float s)
{
    NN_CHECK(settle_zero_for_(dst));
    NN_CHECK(settle_zero_for_(a));
    if (b) NN_CHECK(settle_zero_for_(*b));
    const std::size_t n = dst.size();
    if (pew_ && (pew_->n != n || pew_->full())) NN_CHECK(settle_ew_(true));
    if (!pew_)
    {
        pew_ = std::make_unique<PendingEw>();
        pew_->n = n;
    }
    PendingEw::Op o{};
    o.code = static_cast<EwCode>(code);
    o.op = static_cast<std::uint8_t>(op);
    o.first = first ? 1 : 0;
    o.s = s;
    o.a = pew_->slot(a);
    o.b = b ? pew_->slot(*b) : o.a;
    o.dst = pew_->slot(dst);
    pew_->ops.push_back(o);
    return {};
}

// Launches the recorded calls in order: every Adam / AdamW update chain as one
// nnhip_adam_update pass, any other call with its own kernel. A call is
// skipped when its result is referenced by nobody and read by no later call.
Result<void> HipEngine::settle_ew_(bool keep_adam)
{
    if (!pew_) return keep_adam ? Result<void>{} : flush_adam_();
    std::unique_ptr<PendingEw> g = std::move(pew_);
    const auto& ops = g->ops;
    std::vector<std::ptrdiff_t> last_read(g->slots.size(), -1);
    for (std::size_t i = 0; i < ops.size(); ++i)
    {
        last_read[ops[i].a] = static_cast<std::ptrdiff_t>(i);
        if (PendingEw::reads_b(ops[i])) last_read[ops[i].b] = static_cast<std::ptrdiff_t>(i);
    }
    const auto st = static_cast<hipStream_t>(stream_);
    const std::size_t n = g->n;
    std::size_t i0 = 0;
    if (g->vec_reads)
    {
        NN_TRY(k, swiglu_vec_run_(*g, last_read));
        i0 = k;
        // Any product still recorded whose rows the record reads runs first.
        for (const Tensor& t : g->slots)
            if (std::size_t off = 0; vec_slice_of_(t, off)) NN_CHECK(settle_chain_reads_({&t}));
    }
    for (std::size_t i = i0; i < ops.size();)
    {
        NN_TRY(k, adam_run_(*g, i, last_read));
        if (k)
        {
            i += k;
            continue;
        }
        NN_CHECK(flush_adam_());   // collected updates precede every other launch
        NN_TRY(k2, swiglu_run_(*g, i, last_read));
        if (k2)
        {
            i += k2;
            continue;
        }
        const auto& o = ops[i];
        const Tensor& dst = g->slots[o.dst];
        if (live(dst) || last_read[o.dst] > static_cast<std::ptrdiff_t>(i))
        {
            const float* a = D(g->slots[o.a]);
            const float* b = D(g->slots[o.b]);
            float* out = W(dst);
            switch (o.code)
            {
            case kBin: NN_CHECK(kernel_(nnhip_elementwise_binary(a, b, out, n, o.op, st), "elementwise_binary")); break;
            case kScalar:
                NN_CHECK(kernel_(nnhip_elementwise_binary_scalar(a, out, n, o.op, o.s, o.first, st),
                                 "elementwise_binary_scalar"));
                break;
            case kUnary: NN_CHECK(kernel_(nnhip_elementwise_unary(a, out, n, o.op, st), "elementwise_unary")); break;
            case kAxpy: NN_CHECK(kernel_(nnhip_axpy(a, b, out, n, o.s, st), "axpy_inplace")); break;
            case kCopy:
                NN_CHECK(kernel_(nnhip_copy(a, out, n, st), "clone"));
                break;
            }
        }
        ++i;
    }
    return keep_adam ? Result<void>{} : flush_adam_();
}

// Launches the collected Adam / AdamW updates: one nnhip_adam_update_list call.
Result<void> HipEngine::flush_adam_()
{
    if (padam_.empty()) return {};
    std::vector<PendingAdam> items = std::move(padam_);
    padam_.clear();
    std::vector<float*> p, m, v;
    std::vector<const float*> g;
    std::vector<std::size_t> n;
    for (const auto& a : items)
    {
        p.push_back(W(a.p));
        m.push_back(W(a.m));
        v.push_back(W(a.v));
        g.push_back(D(a.g));
        n.push_back(a.p.size());
    }
    const float* c = padam_args_;
    return kernel_(nnhip_adam_update_list(p.data(), m.data(), v.data(), g.data(), n.data(), items.size(),
                                          c[0] != 0.0f, c[1], c[2], c[3], c[4], c[5], c[6], c[7], c[8], c[9],
                                          static_cast<hipStream_t>(stream_)),
                   "adam update");
}

// True when calls i, i+1, ... of the record are `steps` with one distinct
// buffer per role; slot_of[role] receives the slots.
bool HipEngine::match_run_(const PendingEw& g, std::size_t i, const RunStep* steps, std::size_t len, int nroles,
                           int* slot_of)
{
    if (i + len > g.ops.size()) return false;
    for (int r = 0; r < nroles; ++r) slot_of[r] = -1;
    std::vector<int> role_of(g.slots.size(), -1);
    auto bind = [&](int role, int slot) {
        if (slot_of[role] < 0 && role_of[slot] < 0)
        {
            slot_of[role] = slot;
            role_of[slot] = role;
            return true;
        }
        return slot_of[role] == slot;
    };
    for (std::size_t j = 0; j < len; ++j)
    {
        const RunStep& st = steps[j];
        const PendingEw::Op& o = g.ops[i + j];
        if (!(o.code == st.code && o.op == st.op && o.first == st.first && bind(st.a, o.a) &&
              (st.b < 0 || bind(st.b, o.b)) && bind(st.dst, o.dst)))
            return false;
    }
    return true;
}

// If calls i.. of the record are an Adam(W) update chain whose temporaries
// nobody keeps, launches it as one pass and returns its length; else 0.
Result<std::size_t> HipEngine::adam_run_(const PendingEw& g, std::size_t i,
                                         const std::vector<std::ptrdiff_t>& last_read)
{
    const auto& ops = g.ops;
    for (int decay = 1; decay >= 0; --decay)
    {
        const std::size_t len = kAdamLen + static_cast<std::size_t>(decay);
        int slot_of[kAdamRoles];
        if (!match_run_(g, i, kAdamSteps + (decay ? 0 : 1), len, kAdamRoles, slot_of)) continue;
        bool ok = true;
        for (int r = rG2; ok && r <= rR; ++r)
            ok = !live(g.slots[slot_of[r]]) && last_read[slot_of[r]] < static_cast<std::ptrdiff_t>(i + len);
        if (!ok) continue;
        const PendingEw::Op* c = &ops[i + static_cast<std::size_t>(decay)];   // the first call after the decay
        const float args[10] = {decay ? 1.0f : 0.0f, decay ? ops[i].s : 1.0f, c[0].s, c[1].s, c[2].s, c[4].s,
                                c[7].s, c[9].s, c[11].s, c[13].s};
        const Tensor* mine[4] = {&g.slots[slot_of[rP]], &g.slots[slot_of[rM]], &g.slots[slot_of[rV]],
                                 &g.slots[slot_of[rG]]};
        auto overlap = [](const Tensor& a, const Tensor& b) {
            const float *pa = a.dev_ptr(), *pb = b.dev_ptr();
            return pa && pb && pa < pb + b.size() && pb < pa + a.size();
        };
        bool conflict = !padam_.empty() && std::memcmp(args, padam_args_, sizeof(args)) != 0;
        for (const auto& q : padam_)   // a collected update writing what this one touches, or reading what it writes
            for (const Tensor* t : mine)
                if (overlap(*t, q.p) || overlap(*t, q.m) || overlap(*t, q.v) ||
                    (t != mine[3] && overlap(*t, q.g)))
                    conflict = true;
        if (conflict) NN_CHECK(flush_adam_());
        std::memcpy(padam_args_, args, sizeof(args));
        // The update is launched later, with others: p, m, v and g are held
        // (they are distinct buffers, as match_run_ bound one slot per role).
        padam_.push_back(PendingAdam{g.slots[slot_of[rP]], g.slots[slot_of[rM]], g.slots[slot_of[rV]],
                                     g.slots[slot_of[rG]]});
        // Every kAdamFlush updates go out at once: the GPU updates those
        // tensors while the host records the optimizer's next calls (an AdamW
        // step over 172 tensors is ~2 750 calls, ~2 ms of host time).
        constexpr std::size_t kAdamFlush = 16;
        if (padam_.size() >= kAdamFlush) NN_CHECK(flush_adam_());
        return len;
    }
    return std::size_t{0};
}

// Same for SwiGLU::forward's chain: gate and up read once, s (when kept or
// read later) and out written once.
Result<std::size_t> HipEngine::swiglu_run_(const PendingEw& g, std::size_t i,
                                           const std::vector<std::ptrdiff_t>& last_read)
{
    int slot_of[kSwigluRoles];
    if (!match_run_(g, i, kSwigluSteps, kSwigluLen, kSwigluRoles, slot_of)) return std::size_t{0};
    const auto end = static_cast<std::ptrdiff_t>(i + kSwigluLen);
    for (int r : {sT1, sT2, sT3, sSW})
        if (live(g.slots[slot_of[r]]) || last_read[slot_of[r]] >= end) return std::size_t{0};
    const Tensor& S = g.slots[slot_of[sS]];
    const bool keep_s = live(S) || last_read[slot_of[sS]] >= end;
    NN_CHECK(kernel_(nnhip_swiglu_forward(D(g.slots[slot_of[sG]]), D(g.slots[slot_of[sU]]), keep_s ? W(S) : nullptr,
                                          W(g.slots[slot_of[sO]]), g.n, g.ops[i + 2].s, g.ops[i + 3].s,
                                          static_cast<hipStream_t>(stream_)),
                     "swiglu forward"));
    return kSwigluLen;
}

// SwiGLU::forward's chain at the start of a record whose gate and up are the
// two halves of one recorded matrix-vector product (a token's fc1, and its
// RMSNorm when that is recorded too): both in one nnhip_gemv_swiglu launch,
// bit-identical to the product's launch followed by nnhip_swiglu_forward.
Result<std::size_t> HipEngine::swiglu_vec_run_(const PendingEw& g, const std::vector<std::ptrdiff_t>& last_read)
{
    int slot_of[kSwigluRoles];
    if (!match_run_(g, 0, kSwigluSteps, kSwigluLen, kSwigluRoles, slot_of)) return std::size_t{0};
    const auto end = static_cast<std::ptrdiff_t>(kSwigluLen);
    for (int r : {sT1, sT2, sT3, sSW})
        if (live(g.slots[slot_of[r]]) || last_read[slot_of[r]] >= end) return std::size_t{0};
    const Tensor& G = g.slots[slot_of[sG]];
    const Tensor& U = g.slots[slot_of[sU]];
    std::size_t og = 0, ou = 0;
    PendingMm* r = vec_slice_of_(G, og);
    if (!r || vec_slice_of_(U, ou) != r || og != 0 || ou != G.size() || r->M != 2 * G.size() || g.n != G.size())
        return std::size_t{0};
    // Products of the same input launch together (launch_pending_mm_): not folded then.
    auto partner = [&](const std::unique_ptr<PendingMm>& q) {
        return q && q.get() != r && q->N == 1 && same_t(q->B, r->B);
    };
    if (partner(pmm_)) return std::size_t{0};
    for (const auto& q : pmm_prev_)
        if (partner(q)) return std::size_t{0};
    const bool rms = prms_ && !prms_->bwd && prms_->stage == 6 && same_t(prms_->y, r->B) && r->K <= 1024 &&
                     r->K % 4 == 0 && aligned16(D(r->A));
    std::unique_ptr<PendingMm> o;
    if (pmm_.get() == r)
        o = std::move(pmm_);
    else
        for (std::size_t i = 0; i < pmm_prev_.size(); ++i)
            if (pmm_prev_[i].get() == r)
            {
                o = std::move(pmm_prev_[i]);
                pmm_prev_.erase(pmm_prev_.begin() + static_cast<std::ptrdiff_t>(i));
                break;
            }
    if (merge_of_(o->A)) NN_CHECK(settle_chain_reads_({&o->A}));
    const Tensor& S = g.slots[slot_of[sS]];
    const bool keep_s = live(S) || last_read[slot_of[sS]] >= end;
    float* y = live(o->C) ? W(o->C) : nullptr;
    const float* bias = o->bias.size() ? D(o->bias) : nullptr;
    const auto st = static_cast<hipStream_t>(stream_);
    prof_begin_();
    int rc = 0;
    if (rms)
    {
        std::unique_ptr<PendingRms> q = std::move(prms_);
        const nnhip_gemv_rmsnorm rn{D(q->gamma), q->inv_f, q->eps, W(q->s), W(q->scaled), W(q->var_eps),
                                    W(q->rinv), W(q->normed), W(q->y)};
        rc = nnhip_gemv_swiglu(D(o->A), D(q->x), &rn, bias, y, keep_s ? W(S) : nullptr, W(g.slots[slot_of[sO]]),
                               G.size(), o->K, g.ops[2].s, g.ops[3].s, st);
    }
    else
    {
        NN_CHECK(settle_chain_reads_({&o->B}));
        rc = nnhip_gemv_swiglu(D(o->A), D(o->B), nullptr, bias, y, keep_s ? W(S) : nullptr,
                               W(g.slots[slot_of[sO]]), G.size(), o->K, g.ops[2].s, g.ops[3].s, st);
    }
    prof_end_(o->M, 1, o->K, 1, false, false);
    NN_CHECK(kernel_(rc, "matmul + swiglu (vector)"));
    return kSwigluLen;
}

Result<Tensor> HipEngine::alloc_(std::size_t rows, std::size_t cols)
{
    const std::size_t n = rows * cols;
    if (n == 0) return Tensor(std::shared_ptr<DeviceBuffer>(), rows, cols);
    std::size_t rounded = 0;
    void* p = pool_->alloc(n * sizeof(float), rounded);
    if (!p) return fail("HipEngine: out of device memory allocating " + std::to_string(n * 4) + " bytes");
    return Tensor(std::make_shared<HipBuffer>(pool_, static_cast<float*>(p), n, rounded), rows, cols);
}

Result<std::shared_ptr<DeviceBuffer>> HipEngine::scratch_(std::size_t bytes)
{
    std::size_t rounded = 0;
    void* p = pool_->alloc(bytes < 256 ? 256 : bytes, rounded);
    if (!p) return fail("HipEngine: out of device memory for workspace");
    return std::shared_ptr<DeviceBuffer>(
        std::make_shared<HipBuffer>(pool_, static_cast<float*>(p), rounded / sizeof(float), rounded));
}

Result<void> HipEngine::begin_batch() { return {}; }

Result<void> HipEngine::end_batch()
{
    NN_CHECK(settle());
    return sync_();
}

Result<void> HipEngine::sync_()
{
    const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream_));
    if (e != hipSuccess) return fail(std::string("HipEngine: stream error: ") + hipGetErrorString(e));
    const hipError_t l = hipGetLastError();
    if (l != hipSuccess) return fail(std::string("HipEngine: launch error: ") + hipGetErrorString(l));
    return {};
}

// Submits the recorded work without waiting for it (the reference's CUDA
// engine makes flush_batch a no-op; its Vulkan engine submits the command
// buffer and records on): reads through the engine still wait for what they
// read, and end_batch waits for everything.
Result<void> HipEngine::flush_batch() { return settle(); }

// ── factories and transfers (cpu_engine.hpp:40-72) ─────────────────────────
Tensor HipEngine::create_tensor(std::size_t rows, std::size_t cols)
{
    auto t = alloc_(rows, cols);
    if (!t)
    {
        std::fprintf(stderr, "%s\n", t.error().message.c_str());
        return Tensor(std::shared_ptr<DeviceBuffer>(), 0, 0);
    }
    return *t;
}

// Host data up to kStageSlot bytes goes through a slot of a pinned staging
// ring: the host copy lands in the slot at once and the upload is queued
// behind the work before it, so the call does not wait for the stream (one
// token of incremental inference uploads its ALiBi step bias in every layer).
// A slot is reused only after its last upload has completed (an event per
// slot). Larger data is uploaded and waited for.
Result<bool> HipEngine::upload_(float* dst, const float* src, std::size_t n)
{
    const std::size_t bytes = n * sizeof(float);
    if (bytes > kStageSlot) return false;
    if (!stage_)
    {
        void* p = nullptr;
        if (hipHostMalloc(&p, kStageSlot * kStageSlots, hipHostMallocDefault) != hipSuccess)
        {
            (void)hipGetLastError();
            return false;
        }
        stage_ = p;
        stage_ev_.assign(kStageSlots, nullptr);
        for (void*& e : stage_ev_)
        {
            hipEvent_t ev = nullptr;
            if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess)
                return fail("HipEngine: hipEventCreate failed");
            e = ev;
        }
    }
    const std::size_t slot = stage_next_++ % kStageSlots;
    const auto ev = static_cast<hipEvent_t>(stage_ev_[slot]);
    if (hipEventSynchronize(ev) != hipSuccess) return fail("HipEngine: staging event wait failed");
    char* at = static_cast<char*>(stage_) + slot * kStageSlot;
    std::memcpy(at, src, bytes);
    auto s = static_cast<hipStream_t>(stream_);
    if (hipMemcpyAsync(dst, at, bytes, hipMemcpyHostToDevice, s) != hipSuccess || hipEventRecord(ev, s) != hipSuccess)
        return fail("HipEngine: host to device copy failed");
    return true;
}

Result<Tensor> HipEngine::from_matrix(const Matrix& m)
{
    NN_TRY(t, alloc_(m.rows(), m.cols()));
    if (m.size())
    {
        NN_TRY(queued, upload_(W(t), m.data(), m.size()));
        if (queued) return t;
        auto s = static_cast<hipStream_t>(stream_);
        if (hipMemcpyAsync(W(t), m.data(), m.size() * sizeof(float), hipMemcpyHostToDevice, s) != hipSuccess)
            return fail("from_matrix: host to device copy failed");
        NN_CHECK(sync_());
    }
    return t;
}

Result<Matrix> HipEngine::to_matrix(const Tensor& t)
{
    if (!t.is_gpu()) return fail("to_matrix: tensor is not GPU");
    NN_CHECK(settle_reads_({&t}));
    Matrix m(t.rows(), t.cols());
    if (m.size())
    {
        auto s = static_cast<hipStream_t>(stream_);
        if (hipMemcpyAsync(m.data(), D(t), m.size() * sizeof(float), hipMemcpyDeviceToHost, s) != hipSuccess)
            return fail("to_matrix: device to host copy failed");
    }
    NN_CHECK(sync_());
    return m;
}

Result<void> HipEngine::copy_from(Tensor& dst, const Matrix& src)
{
    if (!dst.is_gpu()) return fail("copy_from: dst tensor is not GPU");
    if (dst.rows() != src.rows() || dst.cols() != src.cols()) return fail("copy_from: shape mismatch");
    NN_CHECK(settle_write_(dst));
    if (src.size())
    {
        NN_TRY(queued, upload_(W(dst), src.data(), src.size()));
        if (queued) return {};
        auto s = static_cast<hipStream_t>(stream_);
        if (hipMemcpyAsync(W(dst), src.data(), src.size() * sizeof(float), hipMemcpyHostToDevice, s) != hipSuccess)
            return fail("copy_from: host to device copy failed");
        NN_CHECK(sync_());
    }
    return {};
}

Result<Tensor> HipEngine::clone(const Tensor& src)
{
    NN_CHECK(check_gpu_({&src}, "clone"));
    NN_CHECK(settle_chain_reads_({&src}));
    NN_TRY(t, alloc_(src.rows(), src.cols()));
    if (src.size()) NN_CHECK(ew_push_(kCopy, 0, false, t, src, nullptr, 0.0f));
    return t;
}

// ── row slices (cpu_engine.hpp:75-114) ──────────────────────────────────────
// Returns a view of src's rows (see unshare_); views of views share the root.
Result<Tensor> HipEngine::slice_rows(const Tensor& src, std::size_t start, std::size_t count)
{
    // A recorded matrix-vector product stays recorded (a read through the
    // slice launches it: PendingMm::yields covers its whole output), so that
    // SwiGLU's chain on a token's fc1 halves can run with it (swiglu_vec_run_).
    if (vec_record_(src))
    {
        NN_CHECK(check_gpu_({&src}, "slice_rows"));
        NN_CHECK(settle_ew_());
    }
    else
        NN_CHECK(need_gpu_({&src}, "slice_rows"));
    if (start + count > src.rows()) return fail("slice_rows: range out of bounds");
    const std::size_t n = count * src.cols();
    if (!n) return alloc_(count, src.cols());
    std::shared_ptr<DeviceBuffer> root = src.device_buffer();
    std::size_t off = start * src.cols();
    if (auto* v = dynamic_cast<HipView*>(root.get()); v && v->aliased())
    {
        off += v->offset();
        root = v->root_ptr();
    }
    auto view = std::make_shared<HipView>(std::move(root), off, n);
    std::erase_if(views_, [](const std::weak_ptr<DeviceBuffer>& w) { return w.expired(); });
    views_.push_back(view);
    if (view_keys_.size() > 4 * views_.size() + 64)   // drop keys of views gone since the last rebuild
    {
        view_keys_.clear();
        for (const auto& w : views_)
            if (auto sp = w.lock())
            {
                view_keys_.insert(sp.get());
                view_keys_.insert(static_cast<HipView*>(sp.get())->root());
            }
    }
    view_keys_.insert(view.get());
    view_keys_.insert(view->root());
    return Tensor(std::static_pointer_cast<DeviceBuffer>(view), count, src.cols());
}

// Before t is written in place: a view t takes its private copy, and every
// live view of t's memory takes one (the copies run before the write on the
// stream; all earlier writes to that memory were launched when the views
// were cut or when they unshared).
Result<void> HipEngine::unshare_(const Tensor& t)
{
    if (views_.empty()) return {};
    const DeviceBuffer* b = t.device_buffer().get();
    if (!b || !view_keys_.count(b)) return {};   // neither a view nor the memory of one
    // A recorded matrix-vector product may still produce the memory (slice_rows
    // leaves it recorded): it runs before the copies are taken.
    NN_CHECK(settle_chain_reads_({&t}));
    auto take_copy = [&](HipView& v) -> Result<void> {
        const std::size_t n = v.capacity();
        NN_TRY(own, alloc_(1, n));
        NN_CHECK(kernel_(nnhip_copy(v.data(), W(own), n, stream_), "slice_rows copy on write"));
        v.materialise(own.device_buffer());
        return {};
    };
    for (auto& w : views_)
        if (auto sp = w.lock())
        {
            auto* v = static_cast<HipView*>(sp.get());
            if (v->aliased() && (v == b || v->root() == b)) NN_CHECK(take_copy(*v));
        }
    std::erase_if(views_, [](const std::weak_ptr<DeviceBuffer>& w) {
        auto sp = w.lock();
        return !sp || !static_cast<HipView*>(sp.get())->aliased();
    });
    view_keys_.clear();
    for (const auto& w : views_)
        if (auto sp = w.lock())
        {
            view_keys_.insert(sp.get());
            view_keys_.insert(static_cast<HipView*>(sp.get())->root());
        }
    return {};
}

// Launches the recorded SwiGLU gradient programs: into their rows of the
// layer's gradient when placed there, and into their own result while that
// is still referenced.
Result<void> HipEngine::settle_swb_()
{
    if (pswb_.empty()) return {};
    std::vector<PendingSwb> rs = std::move(pswb_);
    pswb_.clear();
    if (rs.size() == 2 && rs[0].placed && rs[1].placed && rs[0].up != rs[1].up && !live(rs[0].out) &&
        !live(rs[1].out))
    {
        // The layer's two inserts: both gradients in one pass.
        const PendingSwb& g = rs[0].up ? rs[1] : rs[0];
        const PendingSwb& u = rs[0].up ? rs[0] : rs[1];
        if (same_t(g.G, u.G) && same_t(g.s, u.s) && same_t(g.gate, u.gate))
            return kernel_(nnhip_swiglu_grad_both(D(g.G), D(g.upt), D(g.s), D(g.gate), W(g.dst) + g.off,
                                                  W(u.dst) + u.off, g.out.size(), stream_),
                           "swiglu grad");
    }
    for (auto& r : rs)
    {
        const std::size_t n = r.out.size();
        auto run = [&](float* o) -> Result<void> {
            if (r.up) return kernel_(nnhip_swiglu_grad_up(D(r.G), D(r.gate), D(r.s), o, n, stream_), "swiglu grad up");
            return kernel_(nnhip_swiglu_grad_gate(D(r.G), D(r.upt), D(r.s), D(r.gate), o, n, stream_),
                           "swiglu grad gate");
        };
        if (r.placed) NN_CHECK(run(W(r.dst) + r.off));
        if (live(r.out)) NN_CHECK(run(W(r.out)));
    }
    return {};
}

// A row insert into a tensor whose zero call is still pending does not launch
// the zeroing first: the inserted rows are left out of it (SwiGLU::backward
// zeroes its (2 d_ff, N) gradient and then inserts both halves).
Result<void> HipEngine::insert_rows(Tensor& dst, std::size_t start, const Tensor& src)
{
    NN_CHECK(check_gpu_({&dst, &src}, "insert_rows"));
    if (dst.cols() != src.cols()) return fail("insert_rows: column count mismatch");
    if (start + src.rows() > dst.rows()) return fail("insert_rows: range out of bounds");
    // A recorded SwiGLU gradient inserted into another tensor: written there directly.
    for (std::size_t i = 0; i < pswb_.size(); ++i)
    {
        PendingSwb& r = pswb_[i];
        const std::size_t off = start * dst.cols();
        if (!same_t(r.out, src) || r.placed || r.uses(dst.dev_ptr()) || !aligned16(W(dst) + off)) continue;
        // Records already placed into overlapping rows of dst run first.
        bool overlap = false;
        for (const auto& q : pswb_)
            if (q.placed && same_t(q.dst, dst) && q.off < off + src.size() && off < q.off + q.out.size())
                overlap = true;
        if (overlap) break;
        NN_CHECK(settle_ew_());
        NN_CHECK(settle_chain_write_(dst, true, true));
        for (auto& z : pzero_)
            if (same_t(z.t, dst)) z.covered.emplace_back(start, start + src.rows());
        PendingSwb& q = pswb_[i];
        q.dst = dst;
        q.off = off;
        q.placed = true;
        return {};
    }
    // A recorded transpose of a vector holds its elements in the source's
    // order: the row is copied from the source (a new KV-cache row in
    // incremental inference, compute_layer.hpp:1426-1511).
    const PendingLayout* sl = layout_of_(src);
    const Tensor from = sl && !sl->per_batch && (sl->S.rows() == 1 || sl->S.cols() == 1) ? sl->S : src;
    PendingZero* z = nullptr;
    for (auto& e : pzero_)
        if (same_t(e.t, dst)) z = &e;
    // When that source is a recorded matrix-vector product (the k or v
    // projection), the product writes the row itself when it runs.
    if (!z && src.rows() == 1 && vec_record_(from) && !has_buf(from, dst.dev_ptr()))
    {
        NN_CHECK(settle_ew_());
        NN_CHECK(settle_chain_write_(dst));
        if (PendingMm* r = vec_record_(from); r && !r->uses(dst.dev_ptr()))
        {
            r->out2 = dst;
            r->out2_off = start * dst.cols();
            return {};
        }
    }
    bool src_zero = false;
    for (auto& e : pzero_)
        if (has_buf(e.t, from.dev_ptr())) src_zero = true;
    if (z && !src_zero && !has_buf(from, dst.dev_ptr()))
    {
        NN_CHECK(settle_ew_());
        NN_CHECK(settle_chain_reads_({&from}));
        NN_CHECK(settle_chain_write_(dst, false, true));
        for (auto& e : pzero_)   // (the settles above leave dst's zero record in place)
            if (same_t(e.t, dst)) e.covered.emplace_back(start, start + src.rows());
    }
    else
    {
        NN_CHECK(settle_reads_({&dst, &from}));
        NN_CHECK(settle_write_(dst));
    }
    if (src.size())
        NN_CHECK(kernel_(nnhip_copy(D(from), W(dst) + start * dst.cols(), src.size(), stream_), "insert_rows"));
    return {};
}

// ── gather / scatter (cpu_engine.hpp:125-216) ───────────────────────────────
Result<Tensor> HipEngine::gather_rows(const Tensor& table, const Tensor& indices)
{
    NN_CHECK(need_gpu_({&table, &indices}, "gather_rows"));
    const std::size_t n = indices.size(), D_ = table.cols();
    NN_TRY(out, alloc_(n, D_));
    NN_CHECK(kernel_(nnhip_gather(D(table), D(indices), W(out), table.rows(), D_, n, stream_), "gather_rows"));
    return out;
}

Result<void> HipEngine::scatter_add_rows(Tensor& dst, const Tensor& indices, const Tensor& grad)
{
    NN_CHECK(need_gpu_({&dst, &indices, &grad}, "scatter_add_rows"));
    NN_CHECK(settle_write_(dst));
    if (dst.cols() != grad.cols()) return fail("scatter_add_rows: column count mismatch");
    const std::size_t n = indices.size();
    if (grad.rows() < n) return fail("scatter_add_rows: grad has fewer rows than indices");
    if (n == 0 || dst.cols() == 0) return {};
    NN_TRY(ws, scratch_(nnhip_scatter_add_workspace_bytes(n)));
    return kernel_(nnhip_scatter_add(W(dst), D(indices), D(grad), dst.rows(), dst.cols(), n, ws->data(), stream_),
                   "scatter_add_rows");
}

// ── layout (cpu_engine.hpp:226-287) ─────────────────────────────────────────
Result<Tensor> HipEngine::rearrange_3d(const Tensor& x, std::size_t M, std::size_t B, std::size_t N, bool inverse)
{
    NN_CHECK(check_gpu_({&x}, "rearrange_3d"));
    if (x.size() != M * B * N) return fail("rearrange_3d: element count mismatch");
    // Of a recorded transpose of S (B*N, M): the per-batch transpose of S, recorded too.
    const PendingLayout* t = inverse ? nullptr : layout_of_(x);
    if (t && !t->per_batch && x.rows() == M && x.size() > 0)
    {
        const Tensor S = t->S;
        NN_TRY(out, alloc_(B * M, N));
        NN_CHECK(push_layout_(PendingLayout{S, out, true, M, B, N}));
        return out;
    }
    // Of a recorded Linear output (the attention's head split, compute_layer.hpp
    // AttentionBase::forward): the product writes the heads' layout itself.
    if (!inverse && B > 1 && x.size() > 0)
    {
        PendingMm* r = nullptr;
        if (pmm_ && same_t(x, pmm_->C)) r = pmm_.get();
        for (auto& q : pmm_prev_)
            if (same_t(x, q->C)) r = q.get();
        if (r && r->folded && r->heads.size() && r->heads_B == B && r->heads_N == N && x.rows() == M)
        {
            Tensor out = r->heads;   // written by the group launch of an earlier head split
            r->heads = Tensor();
            return out;
        }
        // Of a recorded W^T G (the attention's output projection backward, then
        // its head split, compute_layer.hpp:1281-1291): the product writes the
        // heads' layout; its own output becomes a recorded merge of those rows,
        // made only if something reads it.
        if (r && !r->folded && r->tA && !r->tB && r->plus.empty() && !r->out2.size() && !r->bias.size() &&
            !r->heads.size() && r->M == M && r->N == B * N && x.rows() == M && B <= 65535)
        {
            NN_CHECK(settle_reads_({&r->A, &r->B}));
            // (settling may have launched the record)
            PendingMm* q = nullptr;
            if (pmm_ && same_t(x, pmm_->C)) q = pmm_.get();
            for (auto& p : pmm_prev_)
                if (same_t(x, p->C)) q = p.get();
            if (q == r)
            {
                NN_TRY(h, alloc_(B * M, N));
                prof_begin_();
                const int rc = nnhip_gemm_heads_ex(D(r->A), D(r->B), nullptr, W(h), M, r->K, B, N, 1, stream_);
                prof_end_(M, N, r->K, B, true, false);
                NN_CHECK(kernel_(rc, "matmul into heads"));
                const Tensor C = r->C;
                if (pmm_ && pmm_.get() == r)
                    pmm_.reset();
                else
                    std::erase_if(pmm_prev_, [r](const std::unique_ptr<PendingMm>& p) { return p.get() == r; });
                NN_CHECK(push_layout_(PendingLayout{h, C, false, M, B, N, true}));
                return h;
            }
        }
        // A launch covers members x B sequences in grid z (at most 65535).
        auto fits = [&](const PendingMm& q) {
            return !q.folded && !q.out2.size() && !q.tA && !q.tB && q.M == M && q.N == B * N && q.K < 1024 &&
                   B <= 65535 &&
                   aligned16(q.A.dev_ptr()) && (!q.bias.size() || aligned16(q.bias.dev_ptr()));
        };
        if (r && fits(*r) && x.rows() == M)
        {
            // The other recorded products of the same input (k and v after q) join the launch.
            std::vector<PendingMm*> grp{r};
            auto join = [&](PendingMm* q) {
                if (q != r && grp.size() < 3 && (grp.size() + 1) * B <= 65535 && fits(*q) && same_t(q->B, r->B) &&
                    q->K == r->K && live(q->C))
                    grp.push_back(q);
            };
            for (auto& q : pmm_prev_) join(q.get());
            if (pmm_) join(pmm_.get());
            for (PendingMm* q : grp) NN_CHECK(settle_reads_({&q->A, &q->B}));
            const float* Ws[3] = {};
            const float* bs[3] = {};
            float* outs[3] = {};
            std::vector<Tensor> hs;
            for (std::size_t i = 0; i < grp.size(); ++i)
            {
                NN_TRY(h, alloc_(B * M, N));
                hs.push_back(h);
                Ws[i] = D(grp[i]->A);
                bs[i] = grp[i]->bias.size() ? D(grp[i]->bias) : nullptr;
                outs[i] = W(h);
            }
            prof_begin_();
            const int rc = nnhip_gemm_heads_group(Ws, D(r->B), bs, outs, grp.size(), M, r->K, B, N, stream_);
            prof_end_(M, N, r->K, B * grp.size(), false, false);
            NN_CHECK(kernel_(rc, "matmul into heads"));
            for (std::size_t i = 0; i < grp.size(); ++i)
            {
                grp[i]->folded = true;
                if (i > 0)
                {
                    grp[i]->heads = hs[i];
                    grp[i]->heads_B = B;
                    grp[i]->heads_N = N;
                }
            }
            return hs[0];
        }
    }
    // The merge of the heads' rows (compute_layer.hpp:1256-1259, 1377-1386):
    // recorded; the products taking it read the rows in place.
    if (inverse && B > 1 && M > 0 && N % 16 == 0 && N > 0 && x.rows() == B * M && aligned16(x.dev_ptr()))
    {
        NN_CHECK(settle_ew_());
        NN_TRY(out, alloc_(M, B * N));
        NN_CHECK(push_layout_(PendingLayout{x, out, false, M, B, N, true}));
        return out;
    }
    NN_CHECK(settle_reads_({&x}));
    NN_TRY(out, alloc_(inverse ? M : B * M, inverse ? B * N : N));
    NN_CHECK(kernel_(nnhip_rearrange_3d(D(x), W(out), M, B, N, inverse ? 1u : 0u, stream_), "rearrange_3d"));
    return out;
}

// Recorded: the two-pass attention reads the source in place; any other read
// of the result launches the copy.
Result<Tensor> HipEngine::transpose(const Tensor& A)
{
    // A recorded matrix-vector product stays recorded (its transpose is the
    // same vector, which insert_rows may take as the product's second
    // destination); making the copy runs it first.
    NN_CHECK(vec_record_(A) ? check_gpu_({&A}, "transpose") : need_gpu_({&A}, "transpose"));
    NN_TRY(out, alloc_(A.cols(), A.rows()));
    if (out.size() == 0) return out;
    NN_CHECK(push_layout_(PendingLayout{A, out, false, 0, 0, 0}));
    return out;
}

// ── GEMM (cpu_engine.hpp:293-419) ───────────────────────────────────────────
Result<Tensor> HipEngine::matmul(const Tensor& A, const Tensor& B, bool tA, bool tB)
{
    // A recorded RMSNorm column as the vector of W x stays recorded: the
    // product normalises it itself when it runs (launch_pending_mm_).
    const bool rms_x = !tA && !tB && B.cols() == 1 && prms_ && !prms_->bwd && prms_->stage == 6 && same_t(prms_->y, B);
    // A recorded merge of heads' rows as A (untransposed) or B stays recorded:
    // the product reads the rows in place (settled here instead).
    const PendingLayout* am = !tA ? merge_of_(A) : nullptr;
    const PendingLayout* bm = merge_of_(B);
    NN_CHECK(check_gpu_({&A, &B}, "matmul"));
    {
        // (copies: settling may change the recorded layouts)
        const Tensor ra = am ? am->S : A, rb = bm ? bm->S : B;
        NN_CHECK(settle_reads_({&ra, rms_x ? nullptr : &rb}));
    }
    const std::size_t M = tA ? A.cols() : A.rows(), K = tA ? A.rows() : A.cols();
    const std::size_t K2 = tB ? B.cols() : B.rows(), N = tB ? B.rows() : B.cols();
    if (K != K2)
        return fail("matmul: dimension mismatch A=" + std::to_string(A.rows()) + "x" + std::to_string(A.cols()) +
                    " B=" + std::to_string(B.rows()) + "x" + std::to_string(B.cols()));
    NN_TRY(C, alloc_(M, N));
    if (!C.size()) return C;
    // Recorded: the Linear layer's next call adds the bias to C or adds C to
    // the weight gradient (compute_layer.hpp Linear), both folded into the
    // product's epilogue; any other use launches the plain product.
    // An earlier record that this product does not read stays recorded (its
    // output may go straight into the heads' layout, see rearrange_3d).
    std::erase_if(pmm_prev_, [](const std::unique_ptr<PendingMm>& r) { return !r->needed(); });
    constexpr std::size_t kKeepPrev = 4;
    if (pmm_ && !pmm_->yields(A.dev_ptr()) && !pmm_->yields(B.dev_ptr()))
    {
        if (pmm_prev_.size() >= kKeepPrev)
        {
            std::unique_ptr<PendingMm> o = std::move(pmm_prev_.front());
            pmm_prev_.erase(pmm_prev_.begin());
            NN_CHECK(launch_pending_mm_(std::move(o)));   // (may take pmm_ into its group)
        }
        if (pmm_) pmm_prev_.push_back(std::move(pmm_));
    }
    else
        NN_CHECK(settle_mm_());
    pmm_ = std::make_unique<PendingMm>(PendingMm{A, B, C, tA, tB, M, N, K, false});
    return C;
}

// Earlier recorded matmuls that read or write p (every one when p is null):
// launched (when still referenced) and dropped. Folded ones are launched only
// when their own output is read or an input written.
Result<void> HipEngine::settle_mm_prev_(const float* p, bool write)
{
    for (std::size_t i = 0; i < pmm_prev_.size();)
    {
        PendingMm& r = *pmm_prev_[i];
        const bool hit = !p || (write ? r.uses(p) : r.yields(p));
        if (!hit)
        {
            ++i;
            continue;
        }
        std::unique_ptr<PendingMm> o = std::move(pmm_prev_[i]);
        pmm_prev_.erase(pmm_prev_.begin() + static_cast<std::ptrdiff_t>(i));
        const std::size_t before = pmm_prev_.size();
        NN_CHECK(launch_pending_mm_(std::move(o)));
        if (pmm_prev_.size() != before) i = 0;   // partners of a grouped launch left the list
    }
    return {};
}

// A recorded matmul whose output is still referenced. A matrix-vector product
// W x (+ bias) launches together with the other recorded ones of the same x
// and shape (the q, k and v Linear forwards of one token in incremental
// inference, compute_layer.hpp:1426-1511): one nnhip_gemv_group launch, the
// same sums as separate launches.
Result<void> HipEngine::launch_pending_mm_(std::unique_ptr<PendingMm> o)
{
    if (!o->needed()) return {};
    auto vec_form = [](const PendingMm& r) {
        return r.N == 1 && r.M > 1 && !r.tA && !r.tB && r.plus.empty() && r.heads.size() == 0 &&
               r.A.cols() == r.K && r.B.cols() == 1;
    };
    if (vec_form(*o))
    {
        std::vector<std::unique_ptr<PendingMm>> grp;
        auto partner = [&](const std::unique_ptr<PendingMm>& q) {
            return q && vec_form(*q) && same_t(q->B, o->B) && q->M == o->M && q->K == o->K && q->needed() &&
                   grp.size() < 3;
        };
        for (std::size_t i = 0; i < pmm_prev_.size();)
            if (partner(pmm_prev_[i]))
            {
                grp.push_back(std::move(pmm_prev_[i]));
                pmm_prev_.erase(pmm_prev_.begin() + static_cast<std::ptrdiff_t>(i));
            }
            else
                ++i;
        if (partner(pmm_)) grp.push_back(std::move(pmm_));
        const bool rms = prms_ && !prms_->bwd && prms_->stage == 6 && same_t(prms_->y, o->B) && o->K <= 1024 &&
                         o->M <= 8192;
        if (!grp.empty() || o->out2.size() || rms)
        {
            grp.insert(grp.begin(), std::move(o));
            const float* R[4] = {};
            const float* bias[4] = {};
            const float* add[4] = {};
            float* y[4] = {};
            float* out[4] = {};
            for (std::size_t i = 0; i < grp.size(); ++i)
            {
                const PendingMm& q = *grp[i];
                if (merge_of_(q.A)) NN_CHECK(settle_chain_reads_({&q.A}));
                R[i] = D(q.A);
                bias[i] = q.bias.size() ? D(q.bias) : nullptr;
                y[i] = live(q.C) ? W(q.C) : nullptr;
                out[i] = q.out2.size() ? W(q.out2) + q.out2_off : nullptr;
                add[i] = q.addx.size() ? D(q.addx) : nullptr;
            }
            prof_begin_();
            int rc = 0;
            if (rms)
            {
                // RMSNorm's outputs come from workgroup (0, 0) of the same launch.
                std::unique_ptr<PendingRms> q = std::move(prms_);
                const nnhip_gemv_rmsnorm rn{D(q->gamma), q->inv_f, q->eps, W(q->s), W(q->scaled), W(q->var_eps),
                                            W(q->rinv), W(q->normed), W(q->y)};
                rc = nnhip_gemv_group_rmsnorm(R, D(q->x), &rn, bias, y, add, out, grp.size(), grp[0]->M, grp[0]->K,
                                              stream_);
            }
            else
            {
                NN_CHECK(settle_chain_reads_({&grp[0]->B}));
                rc = nnhip_gemv_group(R, D(grp[0]->B), bias, y, add, out, grp.size(), grp[0]->M, grp[0]->K, stream_);
            }
            prof_end_(grp[0]->M, 1, grp[0]->K, grp.size(), false, false);
            return kernel_(rc, "matmul (vector group)");
        }
    }
    return launch_mm_(*o, o->C, o->bias.size() ? &o->bias : nullptr, false);
}

// The recorded matmul into `out`: out = A B (+ bias per row) or out += A B;
// with added products, out = sum of A_i^T B_i in one launch.
Result<void> HipEngine::launch_mm_(const PendingMm& r, const Tensor& out, const Tensor* bias, bool accumulate)
{
    if (merge_of_(r.A)) NN_CHECK(settle_chain_reads_({&r.A}));
    // B as heads' rows read in place: the summed input gradient (every B a
    // merge of one shape) and the plain product (the output projection).
    if (const PendingLayout* bm = merge_of_(r.B); bm && !r.tB)
    {
        const PendingLayout l = *bm;
        std::vector<Tensor> Ss{l.S};
        bool all = true;
        for (const auto& [pa, pb] : r.plus)
        {
            const PendingLayout* q = merge_of_(pb);
            all = all && q && q->M == l.M && q->B == l.B && q->N == l.N;
            if (all) Ss.push_back(q->S);
        }
        const bool sum = !r.plus.empty() && all && r.tA && !bias && !accumulate;
        const bool plain = r.plus.empty() && !r.tA;
        if (sum || plain)
        {
            for (const Tensor& t : Ss) NN_CHECK(settle_chain_reads_({&t}));
            const std::size_t n = Ss.size(), Kt = n * r.K;
            const std::size_t wsb = nnhip_gemm_workspace_bytes(r.M, r.N, Kt, 1);
            std::shared_ptr<DeviceBuffer> ws;
            if (wsb)
            {
                NN_TRY(w, scratch_(wsb));
                ws = w;
            }
            int rc;
            prof_begin_();
            if (sum)
            {
                const float* As[3] = {D(r.A)};
                const float* Bs[3] = {};
                for (std::size_t i = 1; i < n; ++i) As[i] = D(r.plus[i - 1].first);
                for (std::size_t i = 0; i < n; ++i) Bs[i] = D(Ss[i]);
                rc = nnhip_gemm_tn_sum_seq(As, Bs, n, W(out), r.M, r.N, r.K, 1.0f, nnhip_by_seq{l.N, l.M * l.N},
                                           ws ? ws->data() : nullptr, wsb, stream_);
                prof_end_(r.M, r.N, Kt, 1, true, false);
            }
            else
            {
                rc = nnhip_gemm_epilogue_seq(D(r.A), D(Ss[0]), W(out), r.M, r.N, r.K, 1.0f, bias ? D(*bias) : nullptr,
                                             accumulate ? 1 : 0, nnhip_by_seq{l.N, l.M * l.N}, ws ? ws->data() : nullptr, wsb,
                                             stream_);
                prof_end_(r.M, r.N, r.K, 1, false, false);
            }
            if (rc != -7) return kernel_(rc, "matmul");
            // (not whole tiles: the merges are made and the product runs as usual)
        }
    }
    for (const auto& [pa, pb] : r.plus) NN_CHECK(settle_chain_reads_({&pb}));
    NN_CHECK(settle_chain_reads_({&r.B}));   // (a recorded RMSNorm column, see matmul)
    if (!r.plus.empty())
    {
        if (bias || accumulate) return fail("matmul: a summed product takes no epilogue");
        const std::size_t n = r.plus.size() + 1, Kt = n * r.K;
        const float* As[3] = {D(r.A)};
        const float* Bs[3] = {D(r.B)};
        for (std::size_t i = 1; i < n; ++i)
        {
            As[i] = D(r.plus[i - 1].first);
            Bs[i] = D(r.plus[i - 1].second);
        }
        const std::size_t wsb = nnhip_gemm_workspace_bytes(r.M, r.N, Kt, 1);
        std::shared_ptr<DeviceBuffer> ws;
        if (wsb)
        {
            NN_TRY(w, scratch_(wsb));
            ws = w;
        }
        prof_begin_();
        const int rc = nnhip_gemm_tn_sum(As, Bs, n, W(out), r.M, r.N, r.K, 1.0f, ws ? ws->data() : nullptr, wsb,
                                         stream_);
        prof_end_(r.M, r.N, Kt, 1, true, false);
        return kernel_(rc, "matmul");
    }
    const std::size_t wsb = nnhip_gemm_workspace_bytes(r.M, r.N, r.K, 1);
    std::shared_ptr<DeviceBuffer> ws;
    if (wsb)
    {
        NN_TRY(w, scratch_(wsb));
        ws = w;
    }
    prof_begin_();
    const int rc = nnhip_gemm_epilogue(D(r.A), D(r.B), W(out), r.A.rows(), r.A.cols(), r.B.rows(), r.B.cols(), r.tA,
                                       r.tB, 1.0f, bias ? D(*bias) : nullptr, accumulate ? 1 : 0,
                                       ws ? ws->data() : nullptr, wsb, stream_);
    prof_end_(r.M, r.N, r.K, 1, r.tA, r.tB);
    return kernel_(rc, "matmul");
}

// The recorded weight-gradient accumulations: one grouped launch (a single
// member as its own product with the accumulating epilogue).
Result<void> HipEngine::settle_acc_()
{
    if (!pacc_) return {};
    std::unique_ptr<PendingAcc> r = std::move(pacc_);
    const std::size_t n = r->mem.size();
    const std::size_t wsb = nnhip_gemm_workspace_bytes(r->M, r->N, r->K, n);
    std::shared_ptr<DeviceBuffer> ws;
    if (wsb)
    {
        NN_TRY(w, scratch_(wsb));
        ws = w;
    }
    const float* As[4] = {};
    const float* Bs[4] = {};
    float* Cs[4] = {};
    float* Rs[4] = {};
    bool all_rs = r->rs_acc >= 0, one_b = true;
    for (std::size_t i = 0; i < n; ++i)
    {
        Cs[i] = W(r->mem[i].second);
        Rs[i] = i < r->rs.size() && r->rs[i].size() ? W(r->rs[i]) : nullptr;
        all_rs = all_rs && Rs[i];
        one_b = one_b && same_t(r->mb[i], r->B);
    }
    // Members' G (A) and input (transposed B) that are merges of heads' rows
    // are read in place (the q, k, v gradients; the output projection's input).
    nnhip_by_seq as[4] = {}, bs[4] = {};
    bool by_seq = false;
    if (r->tB)
        for (std::size_t i = 0; i < n; ++i)
        {
            if (const PendingLayout* q = merge_of_(r->mem[i].first))
            {
                as[i] = nnhip_by_seq{q->N, q->M * q->N};   // rows of q->N per sequence
                const Tensor S = q->S;
                NN_CHECK(settle_chain_reads_({&S}));
                by_seq = true;
            }
            if (const PendingLayout* q = merge_of_(r->mb[i]))
            {
                bs[i] = nnhip_by_seq{q->N, q->M * q->N};
                const Tensor S = q->S;
                NN_CHECK(settle_chain_reads_({&S}));
                by_seq = true;
            }
        }
    int rc = -7;
    if (by_seq)
    {
        for (std::size_t i = 0; i < n; ++i)
        {
            const PendingLayout* qa = as[i].len ? merge_of_(r->mem[i].first) : nullptr;
            const PendingLayout* qb = bs[i].len ? merge_of_(r->mb[i]) : nullptr;
            if ((as[i].len && !qa) || (bs[i].len && !qb)) by_seq = false;   // (made meanwhile)
            As[i] = qa ? D(qa->S) : D(r->mem[i].first);
            Bs[i] = qb ? D(qb->S) : D(r->mb[i]);
        }
        if (by_seq)
        {
            prof_begin_();
            rc = nnhip_gemm_group_acc_seq(As, Bs, Cs, n, r->M, r->N, r->K, r->tB, r->acc ? 1 : 0,
                                          all_rs ? Rs : nullptr, r->rs_acc > 0 ? 1 : 0, as, bs,
                                          ws ? ws->data() : nullptr, wsb, stream_);
            prof_end_(r->M, r->N, r->K, n, false, r->tB);
        }
    }
    if (rc == -7)
    {
        // (no merges, or not whole tiles: the merges are made first)
        for (std::size_t i = 0; i < n; ++i)
        {
            NN_CHECK(settle_chain_reads_({&r->mem[i].first, &r->mb[i]}));
            As[i] = D(r->mem[i].first);
            Bs[i] = D(r->mb[i]);
        }
        prof_begin_();
        rc = one_b ? nnhip_gemm_group_acc(As, D(r->B), Cs, n, r->M, r->N, r->K, r->tB, r->acc ? 1 : 0,
                                          all_rs ? Rs : nullptr, r->rs_acc > 0 ? 1 : 0, ws ? ws->data() : nullptr,
                                          wsb, stream_)
                   : nnhip_gemm_group_acc_each(As, Bs, Cs, n, r->M, r->N, r->K, r->tB, r->acc ? 1 : 0,
                                               all_rs ? Rs : nullptr, r->rs_acc > 0 ? 1 : 0,
                                               ws ? ws->data() : nullptr, wsb, stream_);
        prof_end_(r->M, r->N, r->K, n, false, r->tB);
    }
    NN_CHECK(kernel_(rc, "matmul"));
    if (all_rs) return {};
    // (row sums recorded for some members only: their own launches, of G as a
    // matrix, a merge of heads' rows made first)
    for (std::size_t i = 0; i < n; ++i)
        if (Rs[i])
        {
            NN_CHECK(settle_chain_reads_({&r->mem[i].first}));
            const std::size_t R = r->mem[i].first.rows(), C = r->mem[i].first.cols();
            const float* G = D(r->mem[i].first);
            NN_CHECK(kernel_(r->rs_acc > 0 ? nnhip_reduce_row_sum_add(G, Rs[i], R, C, stream_)
                                           : nnhip_reduce_row(G, Rs[i], R, C, 0u, stream_),
                             "row_reduce_sum"));
        }
    return {};
}

Result<void> HipEngine::settle_mm_()
{
    if (!pmm_) return {};
    return launch_pending_mm_(std::move(pmm_));
}

Result<void> HipEngine::launch_gemm_(const Tensor& A, const Tensor& B, Tensor& C, std::size_t batch, bool tA, bool tB,
                                     Scalar alpha, std::size_t M, std::size_t N, std::size_t K)
{
    // (a deferred scores product of one query may hold its key operand as a recorded transpose)
    NN_CHECK(settle_layout_for_(A));
    NN_CHECK(settle_layout_for_(B));
    const std::size_t wsb = nnhip_gemm_workspace_bytes(M, N, K, batch);
    std::shared_ptr<DeviceBuffer> ws;
    if (wsb)
    {
        NN_TRY(w, scratch_(wsb));
        ws = w;
    }
    prof_begin_();
    const int rc = nnhip_gemm(D(A), D(B), W(C), A.rows(), A.cols(), B.rows(), B.cols(), batch, tA, tB, alpha,
                              ws ? ws->data() : nullptr, wsb, stream_);
    prof_end_(M, N, K, batch, tA, tB);
    return kernel_(rc, "batched_matmul");
}

Result<Tensor> HipEngine::batched_matmul(const Tensor& A, const Tensor& B, std::size_t batch, bool tA, bool tB,
                                         Scalar alpha)
{
    NN_CHECK(check_gpu_({&A, &B}, "batched_matmul"));
    NN_TRY(d0, bdims(A, B, batch, tA, tB, "batched_matmul"));
    NN_TRY(chained, attn_bmm_(A, B, batch, tA, tB, alpha));
    if (chained) return std::move(*chained);
    // The scores of one query per batch entry (incremental inference,
    // compute_layer.hpp:1426-1511) against keys given as a recorded transpose
    // of the KV cache rows: the transpose stays recorded, since the one-query
    // attention reads the cache rows in place; every other reader of the key
    // operand (the GEMM launches, the one-pass kernels) copies it first.
    const PendingLayout* kl = tA && !tB && d0.M == 1 ? layout_of_(B) : nullptr;
    NN_CHECK(kl && !kl->per_batch ? need_gpu_({&A}, "batched_matmul") : need_gpu_({&A, &B}, "batched_matmul"));
    NN_TRY(d, bdims(A, B, batch, tA, tB, "batched_matmul"));
    NN_TRY(C, alloc_(batch * d.M, d.N));
    // The dP product of the attention backward (compute_layer.hpp:1306-1307) is
    // deferred: backward_q / backward_kv recompute its entries where the mask
    // allows them; any other reader gets the full product.
    if (tA && !tB && nnhip_flash_supported(batch, d.M, d.N, d.K, 4) && d.K % 4 == 0)
    {
        NN_CHECK(settle_gemm_());
        pgemm_ = std::make_unique<PendingGemm>(PendingGemm{A, B, C, batch, d.M, d.N, d.K, alpha});
        return C;
    }
    NN_CHECK(launch_gemm_(A, B, C, batch, tA, tB, alpha, d.M, d.N, d.K));
    return C;
}

// ── fused attention (cpu_engine.hpp:426-915) ────────────────────────────────
// Workspace of the attention kernels: mask-cell table, combine counters, partial results.
Result<std::shared_ptr<DeviceBuffer>> HipEngine::attn_ws_(std::size_t batch, std::size_t M, std::size_t N,
                                                          std::size_t K, std::size_t D)
{
    if (batch == 0 || M == 0 || N == 0) return std::shared_ptr<DeviceBuffer>();
    return scratch_(nnhip_bmm_workspace_bytes(batch, M, N, K, D));
}

Result<Tensor> HipEngine::batched_matmul_reduce(const Tensor& A, const Tensor& B, std::size_t batch, ReduceOp op,
                                                bool tA, bool tB, Scalar alpha, bool reduce_cols, const Tensor* mask)
{
    NN_CHECK(need_gpu_({&A, &B, mask}, "batched_matmul_reduce"));
    NN_TRY(d, bdims(A, B, batch, tA, tB, "batched_matmul_reduce"));
    NN_CHECK(mask_ok(mask, d.M, d.N, "batched_matmul_reduce"));
    NN_TRY(out, alloc_(reduce_cols ? batch * d.M : batch, reduce_cols ? 1 : d.N));
    // First call of the forward chain (compute_layer.hpp:1203-1205): deferred.
    if (op == ReduceOp::Max && reduce_cols && tA && !tB && nnhip_flash_supported(batch, d.M, d.N, d.K, 4))
    {
        NN_CHECK(settle_fwd_());
        pfwd_ = std::make_unique<PendingFwd>(PendingFwd{A, B, mask ? std::optional<Tensor>(*mask) : std::nullopt,
                                                        batch, d.M, d.N, d.K, alpha, out, std::nullopt});
        return out;
    }
    NN_TRY(ws, attn_ws_(batch, d.M, d.N, d.K, 1));
    NN_CHECK(kernel_(nnhip_bmm_reduce(D(A), D(B), mask ? D(*mask) : nullptr, W(out), batch, d.M, d.N, d.K, tA, tB,
                                      static_cast<unsigned>(op), alpha, reduce_cols, ws ? ws->data() : nullptr,
                                      stream_),
                     "batched_matmul_reduce"));
    return out;
}

Result<Tensor> HipEngine::batched_matmul_softmax_denom(const Tensor& A, const Tensor& B, const Tensor& row_max,
                                                       std::size_t batch, bool tA, bool tB, Scalar alpha,
                                                       const Tensor* mask)
{
    NN_CHECK(check_gpu_({&A, &B, &row_max, mask}, "batched_matmul_softmax_denom"));
    NN_TRY(d, bdims(A, B, batch, tA, tB, "batched_matmul_softmax_denom"));
    NN_CHECK(vec_ok(row_max, batch * d.M, "batched_matmul_softmax_denom", "row_max"));
    NN_CHECK(mask_ok(mask, d.M, d.N, "batched_matmul_softmax_denom"));
    if (pfwd_ && !pfwd_->l && same_t(row_max, pfwd_->m) && pfwd_->matches(A, B, batch, tA, tB, alpha, mask))
    {
        NN_TRY(l, alloc_(batch * d.M, 1));
        pfwd_->l = l;
        return l;
    }
    NN_CHECK(settle_reads_({&A, &B, &row_max, mask}));
    NN_TRY(out, alloc_(batch * d.M, 1));
    NN_TRY(ws, attn_ws_(batch, d.M, d.N, d.K, 1));
    NN_CHECK(kernel_(nnhip_bmm_softmax_denom(D(A), D(B), D(row_max), mask ? D(*mask) : nullptr, W(out), batch, d.M,
                                             d.N, d.K, tA, tB, alpha, ws ? ws->data() : nullptr, stream_),
                     "batched_matmul_softmax_denom"));
    return out;
}

Result<Tensor> HipEngine::batched_matmul_softmax_apply(const Tensor& A, const Tensor& B, const Tensor& V,
                                                       const Tensor& row_max, const Tensor& denom, std::size_t batch,
                                                       bool tA, bool tB, Scalar alpha, const Tensor* mask)
{
    NN_CHECK(check_gpu_({&A, &B, &V, &row_max, &denom, mask}, "batched_matmul_softmax_apply"));
    if (batch != 0 && V.rows() % batch != 0) return fail("batched_matmul_softmax_apply: rows not divisible by batch");
    NN_TRY(d, bdims(A, B, batch, tA, tB, "batched_matmul_softmax_apply"));
    if (V.rows() / batch != d.N) return fail("batched_matmul_softmax_apply: V rows per batch != N");
    NN_CHECK(vec_ok(row_max, batch * d.M, "batched_matmul_softmax_apply", "row_max"));
    NN_CHECK(vec_ok(denom, batch * d.M, "batched_matmul_softmax_apply", "denom"));
    NN_CHECK(mask_ok(mask, d.M, d.N, "batched_matmul_softmax_apply"));
    // Last call of the forward chain: m, l and O in one pass. V made from Vs
    // (per batch (D, N)) by a recorded rearrange_3d(transpose(Vs), N, batch, D)
    // is read from Vs.
    const bool v_from_chain = pfwd_ && pfwd_->yields(V.dev_ptr());
    const PendingLayout* vl = layout_of_(V);
    const bool v_src = vl && vl->per_batch && vl->B == batch && vl->M == d.N && vl->N == V.cols();
    const Tensor Vs = v_src ? vl->S : V;
    if (!v_from_chain && !v_src) NN_CHECK(settle_reads_({&V}));
    if (!v_from_chain && pfwd_ && pfwd_->l && same_t(row_max, pfwd_->m) && same_t(denom, *pfwd_->l) &&
        pfwd_->matches(A, B, batch, tA, tB, alpha, mask) && nnhip_flash_supported(batch, d.M, d.N, d.K, V.cols()))
    {
        std::unique_ptr<PendingFwd> f = std::move(pfwd_);
        NN_TRY(o, alloc_(batch * d.M, V.cols()));
        NN_TRY(cells, mask_cells_buf_(mask, d.M, d.N));
        // A recorded output also keeps the forward's scores for the backward
        // (one 32 x 32 block per cell, so M and N whole tiles), while all
        // records together hold at most score_budget_ bytes of them. The
        // blocks only save work: when they cannot be had, the backward forms
        // the scores itself.
        Tensor S;
        if (v_src)
        {
            forget_dead_two_();
            constexpr std::size_t kKeep = 64;   // one per layer
            if (ptwo_.size() >= kKeep) ptwo_.erase(ptwo_.begin());
            std::size_t held = 0;
            for (const TwoPassOut& r : ptwo_) held += r.S.size() * sizeof(float);
            if (d.M % 32 == 0 && d.N % 32 == 0 && held + batch * d.M * d.N * sizeof(float) <= score_budget_)
            {
                auto t = alloc_(batch * d.M, d.N);
                if (t) S = *t;
            }
        }
        // The launch waits for others of its shape (the next rows of a
        // document-masked batch) until its results are read.
        if (flash_yields_(D(A)) || flash_yields_(D(B)) || flash_yields_(D(Vs)) || (mask && flash_yields_(D(*mask))) ||
            pflash_.size() >= 2 * NNHIP_FLASH_MAX_ROWS)
            NN_CHECK(settle_flash_());
        PendingFlash r;
        r.Q = A;
        r.K = B;
        r.Vs = Vs;
        r.O = o;
        r.m = f->m;
        r.l = *f->l;
        r.S = S;
        r.mask = mask ? std::optional<Tensor>(*mask) : std::nullopt;
        r.cells = cells;
        r.batch = batch;
        r.M = d.M;
        r.N = d.N;
        r.Kd = d.K;
        r.D = V.cols();
        r.alpha = alpha;
        r.v_dm = v_src;
        pflash_.push_back(std::move(r));
        if (v_src)
            ptwo_.push_back(TwoPassOut{A, B, mask ? std::optional<Tensor>(*mask) : std::nullopt, f->m, *f->l, Vs, o,
                                       batch, alpha, S});
        return o;
    }
    NN_CHECK(settle_reads_({&A, &B, &V, &row_max, &denom, mask}));
    NN_TRY(out, alloc_(batch * d.M, V.cols()));
    NN_TRY(ws, attn_ws_(batch, d.M, d.N, d.K, V.cols()));
    NN_CHECK(kernel_(nnhip_bmm_softmax_apply(D(A), D(B), D(V), D(row_max), D(denom), mask ? D(*mask) : nullptr,
                                             W(out), batch, d.M, d.N, d.K, V.cols(), tA, tB, alpha,
                                             ws ? ws->data() : nullptr, stream_),
                     "batched_matmul_softmax_apply"));
    return out;
}

Result<Tensor> HipEngine::batched_matmul_softmax_backward_q(const Tensor& A, const Tensor& B, const Tensor& P,
                                                            const Tensor& row_max, const Tensor& denom,
                                                            std::size_t batch, bool tA, bool tB, Scalar alpha,
                                                            Tensor& r_out, const Tensor* mask)
{
    NN_CHECK(check_gpu_({&A, &B, &P, &row_max, &denom, mask}, "batched_matmul_softmax_backward_q"));
    NN_TRY(d, bdims(A, B, batch, tA, tB, "batched_matmul_softmax_backward_q"));
    if (P.rows() != batch * d.M || P.cols() != d.N) return fail("batched_matmul_softmax_backward_q: P shape mismatch");
    NN_CHECK(vec_ok(row_max, batch * d.M, "batched_matmul_softmax_backward_q", "row_max"));
    NN_CHECK(vec_ok(denom, batch * d.M, "batched_matmul_softmax_backward_q", "denom"));
    NN_CHECK(mask_ok(mask, d.M, d.N, "batched_matmul_softmax_backward_q"));
    NN_TRY(dq, alloc_(batch * d.K, d.M));
    NN_TRY(r, alloc_(batch * d.M, 1));
    // Middle call of the backward chain on a deferred dP: deferred until backward_kv.
    if (pgemm_ && same_t(P, pgemm_->C) && pgemm_->batch == batch && tA && !tB && d.K % 4 == 0 &&
        nnhip_flash_supported(batch, d.M, d.N, std::max(d.K, pgemm_->K), 4))
    {
        // m and l may still be results of a recorded forward: the backward
        // that consumes this record runs after it.
        NN_CHECK(settle_ew_());
        NN_CHECK(settle_chain_reads_({&A, &B, &row_max, &denom, mask}, true));
        NN_CHECK(settle_bwd_());
        pbwd_ = std::make_unique<PendingBwd>(PendingBwd{A, B, P, row_max, denom,
                                                        mask ? std::optional<Tensor>(*mask) : std::nullopt, batch,
                                                        d.M, d.N, d.K, alpha, dq, r});
        r_out = r;
        return dq;
    }
    NN_CHECK(settle_reads_({&A, &B, &P, &row_max, &denom, mask}));
    NN_TRY(ws, attn_ws_(batch, d.M, d.N, d.K, 1));
    NN_CHECK(kernel_(nnhip_bmm_softmax_backward_q(D(A), D(B), D(P), D(row_max), D(denom), mask ? D(*mask) : nullptr,
                                                  W(dq), W(r), batch, d.M, d.N, d.K, tA, tB, alpha,
                                                  ws ? ws->data() : nullptr, stream_),
                     "batched_matmul_softmax_backward_q"));
    r_out = r;
    return dq;
}

Result<Tensor> HipEngine::batched_matmul_softmax_backward_kv(const Tensor& A, const Tensor& B, const Tensor& P,
                                                             const Tensor& G, const Tensor& R, const Tensor& row_max,
                                                             const Tensor& denom, std::size_t batch, bool tA, bool tB,
                                                             Scalar alpha, Tensor& grad_v_out, const Tensor* mask)
{
    NN_CHECK(check_gpu_({&A, &B, &P, &G, &R, &row_max, &denom, mask}, "batched_matmul_softmax_backward_kv"));
    NN_TRY(d, bdims(A, B, batch, tA, tB, "batched_matmul_softmax_backward_kv"));
    if (P.rows() != batch * d.M || P.cols() != d.N)
        return fail("batched_matmul_softmax_backward_kv: P shape mismatch");
    if (G.rows() != batch * d.M) return fail("batched_matmul_softmax_backward_kv: G rows != batch*M");
    NN_CHECK(vec_ok(R, batch * d.M, "batched_matmul_softmax_backward_kv", "R"));
    NN_CHECK(vec_ok(row_max, batch * d.M, "batched_matmul_softmax_backward_kv", "row_max"));
    NN_CHECK(vec_ok(denom, batch * d.M, "batched_matmul_softmax_backward_kv", "denom"));
    NN_CHECK(mask_ok(mask, d.M, d.N, "batched_matmul_softmax_backward_kv"));
    if (G.cols() < d.K) return fail("batched_matmul_softmax_backward_kv: G cols < K");
    NN_TRY(dk, alloc_(batch * d.K, d.N));
    NN_TRY(dv, alloc_(batch * d.K, d.N));
    // Last call of the backward chain: R, dQ, dK, dV with dP recomputed, never
    // stored. G made from dO (the dP product's left operand) by a recorded
    // rearrange_3d(transpose(dO), M, batch, Kd) is read from dO's columns.
    const bool g_from_chain = (pbwd_ && pbwd_->yields(G.dev_ptr())) || (pgemm_ && pgemm_->yields(G.dev_ptr()));
    const PendingLayout* gl = layout_of_(G);
    const bool g_do = gl && gl->per_batch && pgemm_ && same_t(gl->S, pgemm_->A) && gl->B == batch &&
                      gl->M == d.M && gl->N == pgemm_->K && pgemm_->K == d.K;
    if (!g_from_chain && !g_do) NN_CHECK(settle_reads_({&G}));
    if (!g_from_chain && pbwd_ && pgemm_ && same_t(P, pbwd_->P) && same_t(P, pgemm_->C) && same_t(R, pbwd_->R) &&
        same_t(A, pbwd_->Q) && same_t(B, pbwd_->K) && same_t(row_max, pbwd_->m) && same_t(denom, pbwd_->l) &&
        same_mask(mask, pbwd_->mask) && batch == pbwd_->batch && tA && !tB && alpha == pbwd_->alpha &&
        G.cols() % 4 == 0)
    {
        std::unique_ptr<PendingBwd> q = std::move(pbwd_);
        const PendingGemm& g = *pgemm_;
        NN_TRY(cells, mask_cells_(mask, d.M, d.N));
        // The forward's output from the same inputs (V from g.B): R from it,
        // then one score pass storing dS and dQ from dS.
        std::ptrdiff_t fo = -1;
        for (std::size_t i = 0; g_do && i < ptwo_.size(); ++i)
        {
            const TwoPassOut& r = ptwo_[i];
            if (same_t(r.Q, A) && same_t(r.K, B) && same_t(r.m, row_max) && same_t(r.l, denom) &&
                same_mask(mask, r.mask) && r.batch == batch && r.alpha == alpha && same_t(r.Vs, g.B) &&
                r.O.cols() == d.K)
                fo = static_cast<std::ptrdiff_t>(i);
        }
        if (fo >= 0)
        {
            const TwoPassOut r = std::move(ptwo_[static_cast<std::size_t>(fo)]);
            ptwo_.erase(ptwo_.begin() + fo);
            // Recorded like the forward (the backwards of other rows join it);
            // it reads recorded forwards' results, never a recorded backward's.
            NN_TRY(cbuf, mask_cells_buf_(mask, d.M, d.N));
            bool after_bwd = pflash_.size() >= 2 * NNHIP_FLASH_MAX_ROWS;
            for (const PendingFlash& x : pflash_)
                for (const Tensor* t : {&A, &B, &g.A, &g.B, &r.O, &row_max, &denom, &r.S, mask})
                    after_bwd = after_bwd || (t && x.bwd && x.yields(D(*t)));
            if (after_bwd) NN_CHECK(settle_flash_());
            PendingFlash b;
            b.bwd = true;
            b.Q = A;
            b.K = B;
            b.dO = g.A;
            b.Vs = g.B;
            b.O = r.O;
            b.m = row_max;
            b.l = denom;
            b.S = r.S;
            b.R = q->R;
            b.dQ = q->dQ;
            b.dK = dk;
            b.dV = dv;
            b.mask = mask ? std::optional<Tensor>(*mask) : std::nullopt;
            b.cells = cbuf;
            b.batch = batch;
            b.M = d.M;
            b.N = d.N;
            b.Kd = d.K;
            b.D = d.K;
            b.alpha = alpha;
            b.alpha2 = g.alpha;
            pflash_.push_back(std::move(b));
        }
        else
        {
            NN_CHECK(settle_flash_());   // m and l may come from a recorded forward
            NN_TRY(order, flash_order_(cells, batch, d.M, d.N, 0, 1));
            NN_TRY(ws, scratch_(nnhip_flash_workspace_bytes(batch, d.M, d.N, std::max(d.K, g.K), 4, 1)));
            NN_CHECK(kernel_(nnhip_flash_backward_ordered(D(A), D(B), D(g.A), D(g.B), g_do ? nullptr : D(G),
                                                          g_do ? d.K : G.cols(), mask ? D(*mask) : nullptr, cells,
                                                          D(row_max), D(denom), W(q->R), W(q->dQ), W(dk), W(dv),
                                                          batch, d.M, d.N, d.K, g.K, alpha, g.alpha, 0, g_do ? 1 : 0,
                                                          order, ws->data(), stream_),
                             "batched_matmul_softmax_backward_kv"));
        }
        grad_v_out = dv;
        return dk;
    }
    NN_CHECK(settle_reads_({&A, &B, &P, &G, &R, &row_max, &denom, mask}));
    NN_TRY(ws, attn_ws_(batch, d.M, d.N, d.K, 1));
    NN_CHECK(kernel_(nnhip_bmm_softmax_backward_kv(D(A), D(B), D(P), D(G), D(R), D(row_max), D(denom),
                                                   mask ? D(*mask) : nullptr, W(dk), W(dv), batch, d.M, d.N, d.K,
                                                   G.cols(), tA, tB, alpha, ws ? ws->data() : nullptr, stream_),
                     "batched_matmul_softmax_backward_kv"));
    grad_v_out = dv;
    return dk;
}

// ── column softmax / cross-entropy (cpu_engine.hpp:922-1006) ─────────────────
Result<Tensor> HipEngine::col_softmax_denom(const Tensor& logits, const Tensor& col_max)
{
    NN_CHECK(need_gpu_({&logits, &col_max}, "col_softmax_denom"));
    const std::size_t C = logits.rows(), N = logits.cols();
    if (col_max.rows() != 1 || col_max.cols() != N) return fail("col_softmax_denom: col_max shape mismatch");
    NN_TRY(out, alloc_(1, N));
    NN_TRY(ws, scratch_(nnhip_col_softmax_workspace_bytes(C, N)));
    NN_CHECK(kernel_(nnhip_col_softmax_denom(D(logits), D(col_max), W(out), C, N, ws->data(), stream_),
                     "col_softmax_denom"));
    return out;
}

Result<Tensor> HipEngine::col_softmax_sparse_forward(const Tensor& logits, const Tensor& labels, const Tensor* mask,
                                                     std::size_t vocab, Scalar inv, Tensor& loss_vec_out)
{
    NN_CHECK(check_gpu_({&logits, &labels, mask}, "col_softmax_sparse_forward"));
    // Logits still recorded as a product (the lm_head Linear): the product's
    // epilogue leaves per-tile column statistics, so the logits are read once.
    if (pmm_ && !pmm_->folded && !pmm_->out2.size() && same_t(logits, pmm_->C) &&
        !pmm_->uses(labels.dev_ptr()) &&
        !(mask && pmm_->uses(mask->dev_ptr())) && vocab <= (std::size_t{1} << 24) && vocab <= logits.rows() &&
        labels.rows() == 1 && labels.cols() == logits.cols() && (!mask || (mask->rows() == 1 && mask->cols() == logits.cols())))
    {
        const std::size_t tiles = nnhip_gemm_colstats_tiles(pmm_->M, pmm_->N, pmm_->K, pmm_->tA, pmm_->tB);
        if (tiles)
        {
            NN_CHECK(settle_reads_({&labels, mask}));
            if (pmm_ && same_t(logits, pmm_->C))
            {
                const Tensor a = pmm_->A, b = pmm_->B;   // (merges of heads' rows made)
                NN_CHECK(settle_chain_reads_({&a, &b}));
            }
            if (pmm_ && same_t(logits, pmm_->C))
            {
                std::unique_ptr<PendingMm> r = std::move(pmm_);
                const std::size_t C = logits.rows(), N = logits.cols();
                NN_TRY(stats, scratch_(2 * tiles * N * sizeof(float)));
                NN_TRY(ws, scratch_(2 * N * sizeof(float)));
                prof_begin_();
                const int rc = nnhip_gemm_colstats(D(r->A), D(r->B), W(r->C), r->A.rows(), r->A.cols(), r->B.rows(),
                                                   r->B.cols(), r->tA, r->tB, r->bias.size() ? D(r->bias) : nullptr,
                                                   static_cast<float*>(stats->data()), stream_);
                prof_end_(r->M, r->N, r->K, 1, r->tA, r->tB);
                NN_CHECK(kernel_(rc, "matmul"));
                NN_TRY(grad, alloc_(C, N));
                NN_TRY(lv, alloc_(1, N));
                NN_CHECK(kernel_(nnhip_col_softmax_sparse_from_stats(D(logits), D(labels), mask ? D(*mask) : nullptr,
                                                                      static_cast<const float*>(stats->data()), tiles,
                                                                      W(grad), W(lv), C, N, vocab, inv, ws->data(),
                                                                      stream_),
                                 "col_softmax_sparse_forward"));
                loss_vec_out = lv;
                return grad;
            }
        }
    }
    NN_CHECK(need_gpu_({&logits, &labels, mask}, "col_softmax_sparse_forward"));
    if (vocab > (std::size_t{1} << 24))
        return fail("col_softmax_sparse_forward: vocab_size exceeds 2^24 (float labels not exactly representable)");
    const std::size_t C = logits.rows(), N = logits.cols();
    if (labels.rows() != 1 || labels.cols() != N) return fail("col_softmax_sparse_forward: labels shape mismatch");
    if (vocab > C) return fail("col_softmax_sparse_forward: vocab_size > classes");
    if (mask && (mask->rows() != 1 || mask->cols() != N)) return fail("col_softmax_sparse_forward: mask shape mismatch");
    NN_TRY(grad, alloc_(C, N));
    NN_TRY(lv, alloc_(1, N));
    NN_TRY(ws, scratch_(nnhip_col_softmax_workspace_bytes(C, N)));
    NN_CHECK(kernel_(nnhip_col_softmax_sparse_forward(D(logits), D(labels), mask ? D(*mask) : nullptr, W(grad), W(lv),
                                                      C, N, vocab, inv, ws->data(), stream_),
                     "col_softmax_sparse_forward"));
    loss_vec_out = lv;
    return grad;
}

// ── in-place ops (cpu_engine.hpp:1008-1044) ─────────────────────────────────
// In-place and elementwise calls are recorded (see PendingEw) and run
// together when any other kind of call arrives.
Result<void> HipEngine::add_inplace(Tensor& A, const Tensor& B)
{
    NN_CHECK(check_gpu_({&A, &B}, "add_inplace"));
    if (A.rows() != B.rows() || A.cols() != B.cols()) return fail("add_inplace: shape mismatch");
    if (!A.size()) return {};
    if (pmm_ && !pmm_->folded && !pmm_->bias.size() && pmm_->plus.empty() && !pmm_->out2.size() &&
        same_t(B, pmm_->C) &&
        !pmm_->uses(A.dev_ptr()))
    {
        // Linear backward: the weight-gradient accumulation becomes the
        // product's epilogue (A += product); B stays recorded. A gradient
        // still waiting for zero_grad's fill gets the product written
        // instead (0 + x = x).
        const bool fresh = take_zero_(A);
        NN_CHECK(settle_write_(A));
        if (pmm_ && same_t(B, pmm_->C))
        {
            PendingMm& r = *pmm_;
            r.folded = true;
            // Recorded until the layer's bias row sums of the same G arrive (the
            // launch computes them too); accumulations of one shape run together
            // (the attention's output, q, k and v weight gradients).
            const bool rec = !r.tA && r.plus.empty() && r.M > 1 && r.N > 1 && (r.M * r.N) % 4 == 0 &&
                             aligned16(A.dev_ptr()) && A.size() == r.M * r.N;
            if (rec && pacc_ && pacc_->tB == r.tB && pacc_->M == r.M && pacc_->N == r.N && pacc_->K == r.K &&
                r.B.rows() == pacc_->B.rows() && r.B.cols() == pacc_->B.cols() && pacc_->acc == !fresh &&
                pacc_->mem.size() < 4 && !pacc_->uses(A.dev_ptr()))
            {
                pacc_->mem.emplace_back(r.A, A);
                pacc_->mb.push_back(r.B);
                return {};
            }
            NN_CHECK(settle_acc_());
            if (rec)
            {
                pacc_ = std::make_unique<PendingAcc>(PendingAcc{r.B, r.tB, r.M, r.N, r.K, {}});
                pacc_->acc = !fresh;
                pacc_->mem.emplace_back(r.A, A);
                pacc_->mb.push_back(r.B);
                return {};
            }
            NN_CHECK(launch_mm_(r, A, nullptr, !fresh));
            return {};
        }
        if (fresh) NN_CHECK(zero_now_(A));
    }
    if (prsum_ && !prsum_->folded && same_t(B, prsum_->out) && !prsum_->uses(A.dev_ptr()))
    {
        // A bias / gamma gradient: the row-sum kernel adds its sums into A; B
        // stays recorded. Into a gradient still waiting for its zero fill the
        // sums are written.
        const bool fresh = take_zero_(A);
        NN_CHECK(settle_write_(A));
        if (prsum_ && same_t(B, prsum_->out))
        {
            prsum_->folded = true;
            // The row sums of a recorded weight-gradient product's A (Linear's
            // grad_b += row_reduce_sum(G) after grad_w += G Xᵀ): that launch
            // computes them.
            if (PendingAcc* q = pacc_.get(); q && prsum_->kind == 0 && (q->rs_acc < 0 || q->rs_acc == !fresh) &&
                                             A.rows() == q->M && A.cols() == 1 && !q->uses(A.dev_ptr()))
                for (std::size_t i = 0; i < q->mem.size(); ++i)
                    if (same_t(q->mem[i].first, prsum_->src) && (i >= q->rs.size() || !q->rs[i].size()))
                    {
                        q->rs.resize(q->mem.size());
                        q->rs[i] = A;
                        q->rs_acc = fresh ? 0 : 1;
                        return {};
                    }
            NN_CHECK(launch_rsum_(*prsum_, W(A), !fresh));
            return {};
        }
        if (fresh) NN_CHECK(zero_now_(A));
    }
    // The attention's input gradient (compute_layer.hpp:1397-1408): dx = Wq^T gQ, then dx += Wk^T gK and
    // dx += Wv^T gV, all three products still recorded: dx becomes the sum over K = 3 d_model of one
    // launch (within the GEMM tolerance of the separate products and adds). B stays recorded.
    if (PendingMm *ra = pending_mm_(A), *rb = pending_mm_(B);
        ra && rb && ra != rb && ra->tA && !ra->tB && rb->tA && !rb->tB && ra->M == rb->M && ra->N == rb->N &&
        ra->K == rb->K && ra->K % 16 == 0 && ra->M % 4 == 0 && ra->N % 4 == 0 && rb->plus.empty() &&
        ra->plus.size() < 2 && !ra->bias.size() && !rb->bias.size() && !rb->uses(A.dev_ptr()) &&
        aligned16(rb->A.dev_ptr()) && aligned16(rb->B.dev_ptr()) && aligned16(ra->A.dev_ptr()) &&
        aligned16(ra->B.dev_ptr()))
    {
        ra->plus.emplace_back(rb->A, rb->B);
        rb->folded = true;
        return {};
    }
    NN_CHECK(settle_chain_reads_({&B}));
    NN_CHECK(settle_chain_write_(A));
    return ew_push_(kBin, static_cast<unsigned>(BinaryOp::Add), false, A, A, &B, 0.0f);
}

// The recorded matrix-vector product W x (+ bias) whose output is t and that
// has no second destination yet, if any.
HipEngine::PendingMm* HipEngine::vec_record_(const Tensor& t)
{
    auto ok = [&](PendingMm* r) {
        return r && !r->folded && same_t(r->C, t) && r->N == 1 && r->M > 1 && !r->tA && !r->tB && r->plus.empty() &&
               !r->heads.size() && !r->out2.size() && r->A.cols() == r->K && r->B.cols() == 1;
    };
    if (ok(pmm_.get())) return pmm_.get();
    for (auto& q : pmm_prev_)
        if (ok(q.get())) return q.get();
    return nullptr;
}

// The recorded matrix-vector product (as vec_record_) whose output t is a row
// slice of, with t's offset in it (in floats).
HipEngine::PendingMm* HipEngine::vec_slice_of_(const Tensor& t, std::size_t& off)
{
    const auto* v = dynamic_cast<const HipView*>(t.device_buffer().get());
    if (!v || !v->aliased() || t.cols() != 1) return nullptr;
    auto ok = [&](PendingMm* r) {
        return r && !r->folded && r->N == 1 && r->M > 1 && !r->tA && !r->tB && r->plus.empty() && !r->heads.size() &&
               !r->out2.size() && r->A.cols() == r->K && r->B.cols() == 1 &&
               r->C.device_buffer().get() == v->root();
    };
    PendingMm* r = ok(pmm_.get()) ? pmm_.get() : nullptr;
    for (std::size_t i = 0; !r && i < pmm_prev_.size(); ++i)
        if (ok(pmm_prev_[i].get())) r = pmm_prev_[i].get();
    if (r) off = v->offset();
    return r;
}

// The recorded, not yet folded plain product whose output is t, if any.
HipEngine::PendingMm* HipEngine::pending_mm_(const Tensor& t)
{
    auto ok = [&](PendingMm* r) {
        return r && !r->folded && same_t(r->C, t) && !r->heads.size() && !r->out2.size();
    };
    if (ok(pmm_.get())) return pmm_.get();
    for (auto& q : pmm_prev_)
        if (ok(q.get())) return q.get();
    return nullptr;
}

Result<void> HipEngine::scale_inplace(Tensor& A, Scalar s)
{
    NN_CHECK(check_gpu_({&A}, "scale_inplace"));
    if (!A.size()) return {};
    NN_CHECK(settle_chain_write_(A));
    return ew_push_(kScalar, static_cast<unsigned>(BinaryOp::Mul), false, A, A, nullptr, s);
}

Result<void> HipEngine::axpy_inplace(Tensor& A, Scalar s, const Tensor& B)
{
    NN_CHECK(check_gpu_({&A, &B}, "axpy_inplace"));
    if (A.rows() != B.rows() || A.cols() != B.cols()) return fail("axpy_inplace: shape mismatch");
    if (!A.size()) return {};
    NN_CHECK(settle_chain_reads_({&B}));
    NN_CHECK(settle_chain_write_(A));
    return ew_push_(kAxpy, 0, false, A, A, &B, s);
}

// Consecutive zero calls (Optimizer::zero_grad over every gradient) are
// collected and cleared together, a few launches for all of them.
Result<void> HipEngine::zero(Tensor& A)
{
    NN_CHECK(check_gpu_({&A}, "zero"));
    if (!A.size()) return {};
    NN_CHECK(settle_ew_());
    NN_CHECK(settle_chain_write_(A, false, true));
    for (auto& e : pzero_)
        if (same_t(e.t, A))
        {
            e.covered.clear();
            return {};
        }
    pzero_.push_back(PendingZero{A, {}});
    if (pzero_.size() >= 512) return settle_zero_();
    return {};
}

// The recorded zero calls, or (settle_zero_for_) those whose memory overlaps
// t's: one fill-list launch, rows inserted since the zero call left out.
Result<void> HipEngine::settle_zero_()
{
    if (pzero_.empty()) return {};
    std::vector<PendingZero> ts = std::move(pzero_);
    pzero_.clear();
    return launch_zero_(ts);
}

Result<void> HipEngine::settle_zero_for_(const Tensor& t)
{
    if (pzero_.empty() || !t.dev_ptr() || !t.size()) return {};
    const float *lo = t.dev_ptr(), *hi = lo + t.size();
    std::vector<PendingZero> ts;
    for (std::size_t i = pzero_.size(); i-- > 0;)
    {
        const float* zl = pzero_[i].t.dev_ptr();
        if (zl < hi && lo < zl + pzero_[i].t.size())
        {
            ts.push_back(std::move(pzero_[i]));
            pzero_.erase(pzero_.begin() + static_cast<std::ptrdiff_t>(i));
        }
    }
    return ts.empty() ? Result<void>{} : launch_zero_(ts);
}

// True (and the record dropped) when t itself waits for its zero fill, whole:
// the caller writes all of t instead of adding to it.
bool HipEngine::take_zero_(const Tensor& t)
{
    for (std::size_t i = 0; i < pzero_.size(); ++i)
        if (same_t(pzero_[i].t, t) && pzero_[i].covered.empty())
        {
            pzero_.erase(pzero_.begin() + static_cast<std::ptrdiff_t>(i));
            return true;
        }
    return false;
}

Result<void> HipEngine::zero_now_(const Tensor& t)
{
    std::vector<PendingZero> ts{PendingZero{t, {}}};
    return launch_zero_(ts);
}

Result<void> HipEngine::launch_zero_(std::vector<PendingZero>& ts)
{
    std::vector<float*> ptrs;
    std::vector<std::size_t> counts;
    for (auto& z : ts)
    {
        // Row ranges not covered by inserts since the zero call.
        std::sort(z.covered.begin(), z.covered.end());
        std::size_t row = 0;
        const std::size_t cols = z.t.cols();
        for (const auto& [a, b] : z.covered)
        {
            if (a > row)
            {
                ptrs.push_back(W(z.t) + row * cols);
                counts.push_back((a - row) * cols);
            }
            row = std::max(row, b);
        }
        if (row < z.t.rows())
        {
            ptrs.push_back(W(z.t) + row * cols);
            counts.push_back((z.t.rows() - row) * cols);
        }
    }
    if (ptrs.empty()) return {};
    return kernel_(nnhip_zero_list(ptrs.data(), counts.data(), ptrs.size(), stream_), "zero");
}

// ── reductions (cpu_engine.hpp:1050-1086) ───────────────────────────────────
Result<Tensor> HipEngine::row_reduce_sum(const Tensor& A)
{
    if (const PendingLayout* am = merge_of_(A))
    {
        NN_CHECK(check_gpu_({&A}, "row_reduce_sum"));
        const Tensor S = am->S;
        NN_CHECK(settle_reads_({&S}));
    }
    else
        NN_CHECK(need_gpu_({&A}, "row_reduce_sum"));
    NN_TRY(o, alloc_(A.rows(), 1));
    if (!A.rows()) return o;
    NN_CHECK(settle_rsum_());
    prsum_ = std::make_unique<PendingRowSum>();
    prsum_->src = A;
    prsum_->out = o;
    return o;
}

Result<void> HipEngine::launch_rsum_(const PendingRowSum& r, float* out, bool add)
{
    if (merge_of_(r.src)) NN_CHECK(settle_chain_reads_({&r.src}));
    const std::size_t R = r.src.rows(), C = r.src.cols();
    if (r.kind == 1)
        return kernel_(add ? nnhip_rmsnorm_bwd_rowsum_add(D(r.src), D(r.gamma), D(r.normed), out, R, C, stream_)
                           : nnhip_rmsnorm_bwd_rowsum(D(r.src), D(r.gamma), D(r.normed), out, R, C, stream_),
                       "eval_expr_reduce(rmsnorm backward row sum)");
    return kernel_(add ? nnhip_reduce_row_sum_add(D(r.src), out, R, C, stream_)
                       : nnhip_reduce_row(D(r.src), out, R, C, 0u, stream_),
                   "row_reduce_sum");
}

Result<void> HipEngine::settle_rsum_()
{
    if (!prsum_) return {};
    std::unique_ptr<PendingRowSum> r = std::move(prsum_);
    if (!live(r->out)) return {};
    return launch_rsum_(*r, W(r->out), false);
}
Result<Tensor> HipEngine::row_reduce_max(const Tensor& A)
{
    NN_CHECK(need_gpu_({&A}, "row_reduce_max"));
    NN_TRY(o, alloc_(A.rows(), 1));
    NN_CHECK(kernel_(nnhip_reduce_row(D(A), W(o), A.rows(), A.cols(), 1u, stream_), "row_reduce_max"));
    return o;
}
Result<Tensor> HipEngine::col_reduce_sum(const Tensor& A)
{
    NN_CHECK(need_gpu_({&A}, "col_reduce_sum"));
    NN_TRY(o, alloc_(1, A.cols()));
    NN_TRY(ws, scratch_(nnhip_reduce_col_workspace_bytes(A.rows(), A.cols())));
    NN_CHECK(kernel_(nnhip_reduce_col(D(A), W(o), A.rows(), A.cols(), 0u, ws->data(), stream_), "col_reduce_sum"));
    return o;
}
Result<Tensor> HipEngine::col_reduce_max(const Tensor& A)
{
    NN_CHECK(need_gpu_({&A}, "col_reduce_max"));
    NN_TRY(o, alloc_(1, A.cols()));
    NN_TRY(ws, scratch_(nnhip_reduce_col_workspace_bytes(A.rows(), A.cols())));
    NN_CHECK(kernel_(nnhip_reduce_col(D(A), W(o), A.rows(), A.cols(), 1u, ws->data(), stream_), "col_reduce_max"));
    return o;
}

// ── broadcasts (cpu_engine.hpp:1092-1125) ───────────────────────────────────
Result<void> HipEngine::broadcast_row_inplace(Tensor& A, const Tensor& v, BinaryOp op)
{
    NN_CHECK(check_gpu_({&A, &v}, "broadcast_row_inplace"));
    if (op == BinaryOp::Add && pmm_ && !pmm_->folded && !pmm_->bias.size() && pmm_->plus.empty() &&
        !pmm_->out2.size() && same_t(A, pmm_->C) && v.rows() == A.rows() && v.cols() == 1 && v.size() &&
        !pmm_->uses(v.dev_ptr()))
    {
        // Linear forward: the bias add becomes the product's epilogue. The
        // product stays recorded: when the sparse cross-entropy reads it next
        // (the lm_head logits), its epilogue also yields the column statistics.
        NN_CHECK(settle_reads_({&v}));
        if (pmm_ && same_t(A, pmm_->C))
        {
            pmm_->bias = v;
            return {};
        }
    }
    NN_CHECK(need_gpu_({&A, &v}, "broadcast_row_inplace"));
    NN_CHECK(settle_write_(A));
    if (v.rows() != A.rows() || v.cols() != 1) return fail("broadcast_row_inplace: row_vec shape mismatch");
    return kernel_(nnhip_broadcast_row(D(A), D(v), W(A), A.rows(), A.cols(), static_cast<unsigned>(op), stream_),
                   "broadcast_row_inplace");
}
Result<void> HipEngine::broadcast_col_inplace(Tensor& A, const Tensor& v, BinaryOp op)
{
    NN_CHECK(need_gpu_({&A, &v}, "broadcast_col_inplace"));
    NN_CHECK(settle_write_(A));
    if (v.rows() != 1 || v.cols() != A.cols()) return fail("broadcast_col_inplace: col_vec shape mismatch");
    return kernel_(nnhip_broadcast_col(D(A), D(v), W(A), A.rows(), A.cols(), static_cast<unsigned>(op), stream_),
                   "broadcast_col_inplace");
}

// ── elementwise (cpu_engine.hpp:1131-1266) ──────────────────────────────────
Result<Tensor> HipEngine::elementwise_unary(UnaryOp op, const Tensor& A)
{
    NN_CHECK(check_gpu_({&A}, "elementwise_unary"));
    if (static_cast<unsigned>(op) > static_cast<unsigned>(UnaryOp::Tanh)) return fail("elementwise_unary: bad op");
    if (op == UnaryOp::Rsqrt && prms_ && !prms_->bwd && prms_->stage == 3 && same_t(A, prms_->var_eps))
    {
        NN_TRY(o, alloc_(A.rows(), A.cols()));
        prms_->rinv = o;
        prms_->stage = 4;
        return o;
    }
    // SwiGLU::forward's first call on the gate half of a token's recorded fc1
    // product: the product stays recorded (swiglu_vec_run_ may run it with
    // the chain); the record starts here.
    if (std::size_t off = 1; op == UnaryOp::Neg && A.size() && vec_slice_of_(A, off) && off == 0)
    {
        if (pew_) NN_CHECK(settle_ew_(true));
        NN_TRY(o, alloc_(A.rows(), A.cols()));
        NN_CHECK(ew_push_(kUnary, static_cast<unsigned>(op), false, o, A, nullptr, 0.0f));
        pew_->vec_reads = true;
        return o;
    }
    NN_CHECK(settle_chain_reads_({&A}));
    NN_TRY(o, alloc_(A.rows(), A.cols()));
    if (A.size()) NN_CHECK(ew_push_(kUnary, static_cast<unsigned>(op), false, o, A, nullptr, 0.0f));
    return o;
}
Result<Tensor> HipEngine::elementwise_binary(BinaryOp op, const Tensor& A, const Tensor& B)
{
    NN_CHECK(check_gpu_({&A, &B}, "elementwise_binary"));
    if (A.rows() != B.rows() || A.cols() != B.cols()) return fail("elementwise_binary: shape mismatch");
    if (static_cast<unsigned>(op) > static_cast<unsigned>(BinaryOp::Min)) return fail("elementwise_binary: bad op");
    // x + (W v + bias) of a recorded matrix-vector product (the residual adds of
    // a block in incremental inference, compute_layer.hpp:2413-2437): the
    // product writes the sum as well when it runs (the same rounding).
    if (op == BinaryOp::Add && A.cols() == 1 && A.size() && !has_buf(A, B.dev_ptr()) &&
        (vec_record_(A) || vec_record_(B)))
    {
        const Tensor& X = vec_record_(B) ? A : B;
        const Tensor& Cv = vec_record_(B) ? B : A;
        NN_CHECK(settle_ew_());
        NN_CHECK(settle_chain_reads_({&X}));
        if (PendingMm* r = vec_record_(Cv); r && !r->uses(X.dev_ptr()))
        {
            NN_TRY(o, alloc_(A.rows(), 1));
            r->addx = X;
            r->out2 = o;
            r->out2_off = 0;
            return o;
        }
    }
    // grad + dx of a recorded RMSNorm backward (the residual adds of
    // GPTBlock::backward, compute_layer.hpp:2396, 2404): the layer's pass
    // writes the sum as well (the same rounding).
    if (op == BinaryOp::Add && prms_ && prms_->bwd && prms_->stage == 3 && !same_t(A, B) &&
        (same_t(A, prms_->dx) || same_t(B, prms_->dx)))
    {
        const Tensor& E = same_t(B, prms_->dx) ? A : B;
        if (E.size() && aligned16(E.dev_ptr()) && !prms_->yields(E.dev_ptr()) && !has_buf(E, prms_->dx.dev_ptr()))
        {
            NN_CHECK(settle_ew_());
            NN_CHECK(settle_chain_reads_({&E}));
            if (prms_ && prms_->bwd && prms_->stage == 3 && (same_t(A, prms_->dx) || same_t(B, prms_->dx)))
            {
                std::unique_ptr<PendingRms> q = std::move(prms_);
                const std::size_t F = q->x.rows(), N = q->x.cols();
                NN_TRY(o, alloc_(A.rows(), A.cols()));
                NN_CHECK(kernel_(nnhip_rmsnorm_backward_add(D(q->x), D(q->gamma), D(q->normed), D(q->rinv), q->inv_f,
                                                            W(q->s), W(q->scaled), W(q->dx), D(E), W(o), F, N,
                                                            stream_),
                                 "rmsnorm backward"));
                return o;
            }
        }
    }
    // scores + mask of a deferred scores product (materialised attention): recorded.
    if (op == BinaryOp::Add && pgemm_ && same_t(A, pgemm_->C) && !has_buf(B, A.dev_ptr()) && A.size() &&
        pgemm_->N == B.cols() && pgemm_->K <= 64)
    {
        NN_CHECK(settle_reads_({&B}));
        NN_CHECK(settle_madd_());
        if (pgemm_ && same_t(A, pgemm_->C))
        {
            const PendingGemm& g = *pgemm_;
            NN_TRY(o, alloc_(A.rows(), A.cols()));
            pmadd_ = std::make_unique<PendingMaskAdd>(PendingMaskAdd{g.A, g.B, B, o, g.batch, g.M, g.N, g.K, g.alpha});
            return o;
        }
    }
    // The chain's products with the gate or up half (see elementwise_unary).
    if (op == BinaryOp::Mul && A.size() && pew_ && pew_->vec_reads)
    {
        std::size_t off = 0;
        const bool va = vec_slice_of_(A, off) != nullptr, vb = vec_slice_of_(B, off) != nullptr;
        if (va || vb)
        {
            if (!va) NN_CHECK(settle_chain_reads_({&A}));
            if (!vb) NN_CHECK(settle_chain_reads_({&B}));
            NN_TRY(o, alloc_(A.rows(), A.cols()));
            NN_CHECK(ew_push_(kBin, static_cast<unsigned>(op), false, o, A, &B, 0.0f));
            pew_->vec_reads = true;
            return o;
        }
    }
    NN_CHECK(settle_chain_reads_({&A, &B}));
    NN_TRY(o, alloc_(A.rows(), A.cols()));
    if (A.size()) NN_CHECK(ew_push_(kBin, static_cast<unsigned>(op), false, o, A, &B, 0.0f));
    return o;
}
Result<Tensor> HipEngine::elementwise_binary_scalar(BinaryOp op, const Tensor& A, Scalar s, bool first)
{
    NN_CHECK(check_gpu_({&A}, "elementwise_binary_scalar"));
    if (static_cast<unsigned>(op) > static_cast<unsigned>(BinaryOp::Min))
        return fail("elementwise_binary_scalar: bad op");
    if (prms_ && !first &&
        ((op == BinaryOp::Mul && prms_->stage == 1 && same_t(A, prms_->s)) ||
         (op == BinaryOp::Add && !prms_->bwd && prms_->stage == 2 && same_t(A, prms_->scaled))))
    {
        NN_TRY(o, alloc_(A.rows(), A.cols()));
        if (prms_->stage == 1)
        {
            prms_->scaled = o;
            prms_->inv_f = s;
        }
        else
        {
            prms_->var_eps = o;
            prms_->eps = s;
        }
        ++prms_->stage;
        return o;
    }
    NN_CHECK(settle_chain_reads_({&A}));
    NN_TRY(o, alloc_(A.rows(), A.cols()));
    if (A.size()) NN_CHECK(ew_push_(kScalar, static_cast<unsigned>(op), first, o, A, nullptr, s));
    return o;
}
Result<Tensor> HipEngine::elementwise_select_scalar_cond(CompareOp cmp, const Tensor& A, Scalar sb,
                                                         const Tensor& then_t, Scalar se)
{
    NN_CHECK(need_gpu_({&A, &then_t}, "elementwise_select_scalar_cond"));
    if (A.rows() != then_t.rows() || A.cols() != then_t.cols())
        return fail("elementwise_select: A and then shape mismatch");
    NN_TRY(o, alloc_(A.rows(), A.cols()));
    NN_CHECK(kernel_(nnhip_elementwise_select_scalar_cond(D(A), D(then_t), W(o), A.size(), static_cast<unsigned>(cmp),
                                                          sb, se, stream_),
                     "elementwise_select_scalar_cond"));
    return o;
}

// ── eval_expr (cpu_engine.hpp:1276-1659) ────────────────────────────────────
Result<Tensor> HipEngine::eval_expr(const ExprSpec& spec, std::span<const Tensor> inputs, std::size_t rows,
                                    std::size_t cols)
{
    return eval_impl_(spec, inputs, rows, cols, false);
}
Result<Tensor> HipEngine::eval_expr_reduce(const ExprSpec& spec, std::span<const Tensor> inputs, std::size_t rows,
                                           std::size_t cols)
{
    return eval_impl_(spec, inputs, rows, cols, true);
}

Result<Tensor> HipEngine::eval_impl_(const ExprSpec& spec, std::span<const Tensor> inputs, std::size_t rows,
                                     std::size_t cols, bool vector_out)
{
    NN_CHECK(validate_expr_spec(spec, inputs.size()));
    if (!vector_out)
    {
        NN_TRY(chained, attn_softmax_(spec, inputs, rows, cols));
        if (chained) return std::move(*chained);
    }
    {
        NN_TRY(rms, rms_program_(spec, inputs, rows, cols, vector_out));
        if (rms) return std::move(*rms);
    }
    for (const Tensor& t : inputs)
    {
        if (!t.is_gpu()) return fail("eval_expr: input not GPU");
        NN_CHECK(settle_reads_({&t}));
    }
    const int raxis = vector_out ? expr_spec_reduce_axis(spec) : -1;
    if (vector_out && raxis != 0 && raxis != 1)
        return fail("eval_expr_reduce: expression must reduce along rows or along columns");
    for (std::size_t k = 0; k < inputs.size(); ++k)
    {
        const Tensor& t = inputs[k];
        if (!t.is_gpu()) return fail("eval_expr: input not GPU");
        const ExprView& v = spec.views[k];
        switch (static_cast<ExprViewKind>(v.kind))
        {
        case ExprViewKind::RotateHalf:
            if (t.rows() != rows || t.cols() != cols || v.param == 0 || rows % v.param != 0 || v.param % 2 != 0)
                return fail("eval_expr: RotateHalf shape/param invalid");
            break;
        case ExprViewKind::RowMod:
            if (t.rows() != v.param || t.cols() != cols || v.param == 0 || rows % v.param != 0)
                return fail("eval_expr: RowMod shape/param invalid");
            break;
        case ExprViewKind::RowBroadcast:
            if (t.rows() != rows || t.cols() != 1) return fail("eval_expr: RowBroadcast input must be (rows,1)");
            break;
        case ExprViewKind::ColBroadcast:
            if (t.rows() != 1 || t.cols() != cols) return fail("eval_expr: ColBroadcast input must be (1,cols)");
            break;
        default:
            if (t.rows() != rows || t.cols() != cols) return fail("eval_expr: Linear/reduce input shape mismatch");
            break;
        }
    }
    if (rows * cols == 0) return alloc_(rows, cols);   // the reference returns the (rows, cols) shape here

    if (auto fused = fused_layer_program_(spec, inputs, rows, cols, vector_out)) return std::move(*fused);

    nnhip_expr_program p;
    std::memset(&p, 0, sizeof p);
    p.n_instrs = static_cast<unsigned>(spec.instrs.size());
    p.n_views = static_cast<unsigned>(spec.views.size());
    p.n_consts = static_cast<unsigned>(spec.consts.size());
    p.num_regs = spec.num_regs;
    for (std::size_t i = 0; i < spec.instrs.size(); ++i)
    {
        const ExprInstr& in = spec.instrs[i];
        const unsigned char b[8] = {in.op, in.dst, in.a.kind, in.a.idx, in.b.kind, in.b.idx, in.c.kind, in.c.idx};
        std::memcpy(p.instrs[i], b, 8);
    }
    for (std::size_t k = 0; k < spec.views.size(); ++k)
    {
        p.view_kind[k] = spec.views[k].kind;
        p.view_negate[k] = spec.views[k].negate_first_half;
        p.view_param[k] = spec.views[k].param;
    }
    for (std::size_t c = 0; c < spec.consts.size(); ++c) p.consts[c] = spec.consts[c];
    const float* ptrs[8] = {};
    for (std::size_t k = 0; k < inputs.size(); ++k) ptrs[k] = D(inputs[k]);

    const std::size_t orow = vector_out ? (raxis == 0 ? rows : 1) : rows;
    const std::size_t ocol = vector_out ? (raxis == 0 ? 1 : cols) : cols;
    NN_TRY(o, alloc_(orow, ocol));
    NN_TRY(ws, scratch_(nnhip_eval_expr_workspace_bytes(&p, rows, cols)));
    const int rc = nnhip_eval_expr(&p, ptrs, W(o), rows, cols, vector_out ? 1 : 0, ws->data(), stream_);
    if (rc == -4)
        return fail("eval_expr_reduce: output chain reads an input directly; the output is not constant along "
                    "the reduced axis");
    NN_CHECK(kernel_(rc, "eval_expr"));
    return o;
}

// RMSNorm::forward's programs: the sum of squares starts a PendingRms, the
// normalize continues it and the scale runs the whole forward in one pass.
Result<std::optional<Tensor>> HipEngine::rms_program_(const ExprSpec& spec, std::span<const Tensor> inputs,
                                                      std::size_t rows, std::size_t cols, bool vector_out)
{
    using R = std::optional<Tensor>;
    const float* a[5] = {};
    auto input = [&](const float* p) -> const Tensor* {
        for (const Tensor& t : inputs)
            if (t.dev_ptr() == p) return &t;
        return nullptr;
    };
    if (vector_out && inputs.size() >= 3 && bind(canon(LayerProg::RmsBwdColSum), spec, inputs, a))
    {
        const Tensor *g = input(a[0]), *gamma = input(a[1]), *nrm = input(a[2]);
        if (!g || !gamma || !nrm || !g->is_gpu() || g->rows() != rows || g->cols() != cols ||
            nrm->rows() != rows || nrm->cols() != cols || gamma->rows() != rows || gamma->cols() != 1 ||
            rows == 0 || rows > 1024 || cols == 0 || cols % 4 != 0 || !aligned16(a[0]) || !aligned16(a[2]))
            return R();
        NN_CHECK(settle_rms_());
        NN_CHECK(settle_reads_({g, gamma, nrm}));
        NN_TRY(o, alloc_(1, cols));
        prms_ = std::make_unique<PendingRms>();
        prms_->bwd = true;
        prms_->x = *g;
        prms_->gamma = *gamma;
        prms_->normed = *nrm;
        prms_->s = o;
        return R(o);
    }
    if (!vector_out && prms_ && prms_->bwd && prms_->stage == 2 && inputs.size() >= 5 &&
        bind(canon(LayerProg::RmsBwdDx), spec, inputs, a))
    {
        PendingRms& r = *prms_;
        const Tensor* rinv = input(a[4]);
        if (a[0] != r.x.dev_ptr() || a[1] != r.gamma.dev_ptr() || a[2] != r.scaled.dev_ptr() ||
            a[3] != r.normed.dev_ptr() || !rinv || rinv->rows() != 1 || rinv->cols() != cols ||
            r.x.rows() != rows || r.x.cols() != cols || !aligned16(a[4]) || r.uses(a[4]))
            return R();
        NN_CHECK(settle_reads_({rinv}));
        if (!prms_ || !prms_->bwd || prms_->stage != 2) return R();
        // Recorded: the block's residual add of dx that usually follows
        // (elementwise_binary) runs in the same pass.
        NN_TRY(o, alloc_(rows, cols));
        prms_->rinv = *rinv;
        prms_->dx = o;
        prms_->stage = 3;
        return R(o);
    }
    if (vector_out)
    {
        if (inputs.size() < 1 || !bind(canon(LayerProg::RmsSumSq), spec, inputs, a)) return R();
        const Tensor& x = inputs[0];
        // float4 kernels for N % 4 == 0; narrow ones otherwise (one token's (F, 1) activations)
        const bool narrow = cols % 4 != 0 && cols <= 65535;
        if (!x.is_gpu() || a[0] != x.dev_ptr() || x.rows() != rows || x.cols() != cols || rows == 0 ||
            rows > 1024 || cols == 0 || (!narrow && (cols % 4 != 0 || !aligned16(a[0]))))
            return R();
        NN_CHECK(settle_rms_());
        // x = a + b still recorded as the last elementwise call (the block's
        // residual add, GPTBlock::forward): the layer's pass forms and writes x.
        Tensor xa, xb;
        if (!narrow && pew_ && !pew_->ops.empty())
        {
            const PendingEw::Op& e = pew_->ops.back();
            const Tensor& d = pew_->slots[e.dst];
            std::size_t refs = 0;
            for (const auto& op : pew_->ops)
                refs += (op.dst == e.dst) + (op.a == e.dst) + (PendingEw::reads_b(op) && op.b == e.dst);
            if (e.code == kBin && e.op == static_cast<std::uint8_t>(BinaryOp::Add) && same_t(d, x) && refs == 1 &&
                e.a != e.dst && e.b != e.dst)
            {
                const Tensor &ta = pew_->slots[e.a], &tb = pew_->slots[e.b];
                if (ta.rows() == rows && ta.cols() == cols && tb.rows() == rows && tb.cols() == cols &&
                    aligned16(ta.dev_ptr()) && aligned16(tb.dev_ptr()) && !has_buf(ta, x.dev_ptr()) &&
                    !has_buf(tb, x.dev_ptr()))
                {
                    xa = ta;
                    xb = tb;
                    pew_->ops.pop_back();
                    if (pew_->ops.empty()) pew_.reset();
                }
            }
        }
        NN_CHECK(settle_reads_(xa.size() ? std::initializer_list<const Tensor*>{&xa, &xb}
                                         : std::initializer_list<const Tensor*>{&x}));
        NN_TRY(o, alloc_(1, cols));
        prms_ = std::make_unique<PendingRms>();
        prms_->x = x;
        prms_->xa = xa;
        prms_->xb = xb;
        prms_->s = o;
        return R(o);
    }
    if (!prms_ || prms_->bwd || inputs.size() < 2) return R();
    PendingRms& r = *prms_;
    if (r.x.rows() != rows || r.x.cols() != cols) return R();
    if (r.stage == 4 && bind(canon(LayerProg::RmsNormalize), spec, inputs, a) && a[0] == r.x.dev_ptr() &&
        a[1] == r.rinv.dev_ptr())
    {
        NN_TRY(o, alloc_(rows, cols));
        r.normed = o;
        r.stage = 5;
        return R(o);
    }
    if (r.stage == 5 && bind(canon(LayerProg::RmsScale), spec, inputs, a) && a[0] == r.normed.dev_ptr() &&
        (aligned16(a[1]) || cols % 4 != 0))
    {
        const Tensor* gamma = nullptr;
        for (const Tensor& t : inputs)
            if (t.dev_ptr() == a[1]) gamma = &t;
        if (!gamma || gamma->rows() != rows || gamma->cols() != 1 || prms_->uses(a[1])) return R();
        NN_CHECK(settle_reads_({gamma}));
        if (!prms_ || prms_->stage != 5) return R();
        if (cols == 1 && rows <= 1024)
        {
            // One token's column: recorded, so that the matrix-vector products
            // reading it can normalise it themselves (launch_pending_mm_).
            NN_TRY(o, alloc_(rows, cols));
            prms_->gamma = *gamma;
            prms_->y = o;
            prms_->stage = 6;
            return R(o);
        }
        std::unique_ptr<PendingRms> q = std::move(prms_);
        NN_TRY(o, alloc_(rows, cols));
        if (q->xa.size())
        {
            NN_CHECK(settle_reads_({&q->xa, &q->xb}));
            NN_CHECK(kernel_(nnhip_rmsnorm_forward_sum(D(q->xa), D(q->xb), W(q->x), D(*gamma), q->inv_f, q->eps,
                                                       W(q->s), W(q->scaled), W(q->var_eps), W(q->rinv),
                                                       W(q->normed), W(o), rows, cols, stream_),
                             "rmsnorm forward"));
            return R(o);
        }
        NN_CHECK(kernel_(nnhip_rmsnorm_forward(D(q->x), D(*gamma), q->inv_f, q->eps, W(q->s), W(q->scaled),
                                               W(q->var_eps), W(q->rinv), W(q->normed), W(o), rows, cols, stream_),
                         "rmsnorm forward"));
        return R(o);
    }
    return R();
}

// The recorded RMSNorm calls so far, with their separate kernels.
Result<void> HipEngine::settle_rms_()
{
    if (!prms_) return {};
    std::unique_ptr<PendingRms> r = std::move(prms_);
    const std::size_t F = r->x.rows(), N = r->x.cols();
    if (r->bwd && r->stage == 3)
        return kernel_(nnhip_rmsnorm_backward(D(r->x), D(r->gamma), D(r->normed), D(r->rinv), r->inv_f, W(r->s),
                                              W(r->scaled), W(r->dx), F, N, stream_),
                       "rmsnorm backward");
    if (r->bwd)
    {
        NN_CHECK(kernel_(nnhip_rmsnorm_bwd_colsum(D(r->x), D(r->gamma), D(r->normed), W(r->s), F, N, stream_),
                         "eval_expr_reduce(rmsnorm backward column sum)"));
        if (r->stage >= 2)
            NN_CHECK(kernel_(nnhip_elementwise_binary_scalar(D(r->s), W(r->scaled), N,
                                                             static_cast<unsigned>(BinaryOp::Mul), r->inv_f, 0, stream_),
                             "elementwise_binary_scalar"));
        return {};
    }
    if (r->xa.size())
    {
        // the residual add first, then the calls recorded so far
        NN_CHECK(settle_reads_({&r->xa, &r->xb}));
        NN_CHECK(kernel_(nnhip_elementwise_binary(D(r->xa), D(r->xb), W(r->x), r->x.size(),
                                                  static_cast<unsigned>(BinaryOp::Add), stream_),
                         "elementwise_binary"));
    }
    if (r->stage == 6)
        return kernel_(nnhip_rmsnorm_forward(D(r->x), D(r->gamma), r->inv_f, r->eps, W(r->s), W(r->scaled),
                                             W(r->var_eps), W(r->rinv), W(r->normed), W(r->y), F, N, stream_),
                       "rmsnorm forward");
    NN_CHECK(kernel_(nnhip_rmsnorm_sumsq(D(r->x), W(r->s), F, N, stream_), "eval_expr_reduce(rmsnorm sum of squares)"));
    if (r->stage >= 2)
        NN_CHECK(kernel_(nnhip_elementwise_binary_scalar(D(r->s), W(r->scaled), N, static_cast<unsigned>(BinaryOp::Mul),
                                                         r->inv_f, 0, stream_),
                         "elementwise_binary_scalar"));
    if (r->stage >= 3)
        NN_CHECK(kernel_(nnhip_elementwise_binary_scalar(D(r->scaled), W(r->var_eps), N,
                                                         static_cast<unsigned>(BinaryOp::Add), r->eps, 0, stream_),
                         "elementwise_binary_scalar"));
    if (r->stage >= 4)
        NN_CHECK(kernel_(nnhip_elementwise_unary(D(r->var_eps), W(r->rinv), N, static_cast<unsigned>(UnaryOp::Rsqrt),
                                                 stream_),
                         "elementwise_unary"));
    if (r->stage >= 5)
        NN_CHECK(kernel_(nnhip_colbcast_mul(D(r->x), D(r->rinv), W(r->normed), F, N, stream_),
                         "eval_expr(rmsnorm normalize)"));
    return {};
}

// Softmax rows of a recorded scores + mask (the attention probabilities), and
// the softmax backward of such probabilities against a deferred dO^T V
// product: both recorded for the one-pass kernels.
Result<std::optional<Tensor>> HipEngine::attn_softmax_(const ExprSpec& spec, std::span<const Tensor> inputs,
                                                       std::size_t rows, std::size_t cols)
{
    using R = std::optional<Tensor>;
    const float* a[5] = {};
    auto tensor_of = [&](const float* p) -> const Tensor* {
        for (const Tensor& t : inputs)
            if (t.dev_ptr() == p) return &t;
        return nullptr;
    };
    if (pmadd_ && inputs.size() >= 1 && same_t(inputs[0], pmadd_->out) && rows == pmadd_->out.rows() &&
        cols == pmadd_->out.cols() && bind(canon(LayerProg::SoftmaxFwd), spec, inputs, a))
    {
        const PendingMaskAdd& r = *pmadd_;
        if (!nnhip_flash_supported(r.batch, r.M, r.N, r.Kd, 4) || r.Kd % 4 != 0) return R();
        if (r.mask.rows() != r.batch * r.M && r.mask.rows() != r.M) return R();
        forget_dead_attn_();
        NN_TRY(A, alloc_(rows, cols));
        auto p = std::make_shared<PendingAttn>();
        p->Q = r.Q;
        p->K = r.K;
        p->mask = r.mask;
        p->A = A;
        p->batch = r.batch;
        p->M = r.M;
        p->N = r.N;
        p->Kd = r.Kd;
        p->alpha = r.alpha;
        pattn_.push_back(std::move(p));
        return R(A);
    }
    if (inputs.size() >= 2 && pgemm_ && bind(canon(LayerProg::SoftmaxBwd), spec, inputs, a))
    {
        const Tensor* y = tensor_of(a[0]);
        const Tensor* g = tensor_of(a[1]);
        auto p = y ? attn_of_(*y) : nullptr;
        if (!p || !g || !p->stats || !same_t(*g, pgemm_->C)) return R();
        const PendingGemm& pg = *pgemm_;
        if (pg.batch != p->batch || pg.M != p->M || pg.N != p->N || pg.K != p->Kd) return R();
        NN_CHECK(settle_ds_());
        NN_TRY(out, alloc_(rows, cols));
        pds_ = std::make_unique<PendingDs>(PendingDs{p, pg.A, pg.B, out, pg.K, pg.alpha});
        return R(out);
    }
    return R();
}

// Fused kernels for the layer programs (k_fused.hip, k_softmax.hip). Returns
// nullopt when the program, its bindings or its shape are not one of those;
// the generic interpreter then evaluates it.
std::optional<Result<Tensor>> HipEngine::fused_layer_program_(const ExprSpec& spec, std::span<const Tensor> inputs,
                                                              std::size_t rows, std::size_t cols, bool vector_out)
{
    const float* a[5] = {};
    auto is = [&](LayerProg p) { return bind(canon(p), spec, inputs, a); };
    const bool vec4 = cols % 4 == 0;
    auto run = [&](std::size_t orow, std::size_t ocol, auto&& launch, const char* what) -> Result<Tensor> {
        NN_TRY(o, alloc_(orow, ocol));
        NN_CHECK(kernel_(launch(W(o)), what));
        return o;
    };
    if (!vector_out)
    {
        if (is(LayerProg::SoftmaxFwd))
            return run(rows, cols, [&](float* o) { return nnhip_row_softmax(a[0], o, rows, cols, stream_); },
                       "eval_expr(softmax)");
        if (is(LayerProg::SoftmaxBwd))
            return run(rows, cols,
                       [&](float* o) { return nnhip_row_softmax_backward(a[0], a[1], o, rows, cols, stream_); },
                       "eval_expr(softmax backward)");
        if (!vec4) return std::nullopt;
        if (is(LayerProg::RmsNormalize))
            return run(rows, cols, [&](float* o) { return nnhip_colbcast_mul(a[0], a[1], o, rows, cols, stream_); },
                       "eval_expr(rmsnorm normalize)");
        if (is(LayerProg::RmsScale))
            return run(rows, cols, [&](float* o) { return nnhip_rowbcast_mul(a[0], a[1], o, rows, cols, stream_); },
                       "eval_expr(rmsnorm scale)");
        if (is(LayerProg::RmsBwdDx))
            return run(rows, cols,
                       [&](float* o) {
                           return nnhip_rmsnorm_bwd_dx(a[0], a[1], a[2], a[3], a[4], o, rows, cols, stream_);
                       },
                       "eval_expr(rmsnorm backward dx)");
        // The SwiGLU gradients are recorded (PendingSwb) when their operands
        // allow the float4 kernels; the layer's next calls insert them.
        auto arg = [&](const float* p) -> Tensor {
            for (const Tensor& t : inputs)
                if (t.dev_ptr() == p) return t;
            return Tensor();
        };
        const bool al = aligned16(a[0]) && aligned16(a[1]) && aligned16(a[2]);
        if (is(LayerProg::SwigluGate) && al && aligned16(a[3]))
        {
            if (pswb_.size() >= 2) NN_CHECK(settle_swb_());
            NN_TRY(o, alloc_(rows, cols));
            PendingSwb r;
            r.up = false;
            r.G = arg(a[0]);
            r.upt = arg(a[1]);
            r.s = arg(a[2]);
            r.gate = arg(a[3]);
            r.out = o;
            pswb_.push_back(std::move(r));
            return Result<Tensor>(o);
        }
        if (is(LayerProg::SwigluUp) && al)
        {
            if (pswb_.size() >= 2) NN_CHECK(settle_swb_());
            NN_TRY(o, alloc_(rows, cols));
            PendingSwb r;
            r.up = true;
            r.G = arg(a[0]);
            r.gate = arg(a[1]);
            r.s = arg(a[2]);
            r.out = o;
            pswb_.push_back(std::move(r));
            return Result<Tensor>(o);
        }
        return std::nullopt;
    }
    if (!vec4) return std::nullopt;
    if (is(LayerProg::RmsSumSq))
        return run(1, cols, [&](float* o) { return nnhip_rmsnorm_sumsq(a[0], o, rows, cols, stream_); },
                   "eval_expr_reduce(rmsnorm sum of squares)");
    if (is(LayerProg::RmsBwdColSum))
        return run(1, cols,
                   [&](float* o) { return nnhip_rmsnorm_bwd_colsum(a[0], a[1], a[2], o, rows, cols, stream_); },
                   "eval_expr_reduce(rmsnorm backward column sum)");
    if (is(LayerProg::RmsBwdRowSum))
    {
        const Tensor *g = nullptr, *gm = nullptr, *nm = nullptr;
        for (const Tensor& t : inputs)
        {
            if (t.dev_ptr() == a[0]) g = &t;
            if (t.dev_ptr() == a[1]) gm = &t;
            if (t.dev_ptr() == a[2]) nm = &t;
        }
        if (g && gm && nm && aligned16(a[0]) && aligned16(a[2]))
        {
            NN_CHECK(settle_rsum_());
            NN_TRY(o, alloc_(rows, 1));
            prsum_ = std::make_unique<PendingRowSum>();
            prsum_->src = *g;
            prsum_->gamma = *gm;
            prsum_->normed = *nm;
            prsum_->kind = 1;
            prsum_->out = o;
            return Result<Tensor>(o);
        }
        return run(rows, 1,
                   [&](float* o) { return nnhip_rmsnorm_bwd_rowsum(a[0], a[1], a[2], o, rows, cols, stream_); },
                   "eval_expr_reduce(rmsnorm backward row sum)");
    }
    return std::nullopt;
}

} // namespace nn
