// ORACLE — test infrastructure only. Nothing in the product links this.
//
// cpu_algebra.hpp — the CPU arithmetic under the CpuEngine restatement:
// a block-parallel thread pool and the 64-blocked GEMM / transpose /
// row- and column-reductions of the reference's Matrix.
//
// Followed from (paths under /root/reference):
//   thread pool, caller participates   include/neuralnet.cpp/core_threadpool.hpp:26-612
//   PARALLEL_THRESHOLD = 524288        include/neuralnet.cpp/config.hpp:44
//   BLOCK_SIZE = 64                    include/neuralnet.cpp/config.hpp:22
//   blocked GEMM NN / NT / TN          include/neuralnet.cpp/algebra_matrix.hpp:173-350, 354-660
//     (per (i-block, j-block) task; for each 64-wide k block the B block is
//      copied transposed into a stack tile, each C element gets the k-block's
//      partial dot added: C[i][j] += sum_kk A[i][k0+kk] * B[k0+kk][j])
//   blocked transpose                  include/neuralnet.cpp/algebra_matrix.hpp:121-169
//   row_reduce (per row, serial in c)  include/neuralnet.cpp/algebra_matrix.hpp:801-826
//   col_reduce (row-block partials)    include/neuralnet.cpp/algebra_matrix.hpp:836-900
// The reference vectorises the k-block dot with `#pragma clang loop
// vectorize(assume_safety)`, i.e. with compiler-chosen reassociation; here the
// dot is split into 8 interleaved partial sums (an 8-lane vector order). The
// result differs from the reference only in rounding.
#pragma once

#include <algorithm>
#include <array>
#include <atomic>
#include <condition_variable>
#include <cstddef>
#include <cstdlib>
#include <functional>
#include <mutex>
#include <span>
#include <thread>
#include <vector>

namespace nn::oracle
{

inline constexpr std::size_t BLOCK = 64;
inline constexpr std::size_t PARALLEL_THRESHOLD = 524288;

// Fixed-size pool; parallel_for(n, f) runs f(0..n-1) with the caller
// participating, returning when every index is done.
class ThreadPool
{
public:
    explicit ThreadPool(std::size_t n)
    {
        for (std::size_t i = 1; i < n; ++i)
            workers_.emplace_back([this] { loop_(); });
    }
    ~ThreadPool()
    {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
            ++gen_;
        }
        cv_.notify_all();
        for (auto& t : workers_)
            t.join();
    }
    [[nodiscard]] std::size_t size() const noexcept { return workers_.size() + 1; }

    void parallel_for(std::size_t n, const std::function<void(std::size_t)>& f)
    {
        if (n == 0) return;
        if (n == 1 || workers_.empty())
        {
            for (std::size_t i = 0; i < n; ++i) f(i);
            return;
        }
        std::unique_lock<std::mutex> call(call_mu_);
        {
            std::lock_guard<std::mutex> lk(mu_);
            job_ = &f;
            job_n_ = n;
            next_.store(0);
            pending_ = workers_.size();
            ++gen_;
        }
        cv_.notify_all();
        run_();
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [this] { return pending_ == 0; });
        job_ = nullptr;
    }

private:
    void run_()
    {
        for (;;)
        {
            const std::size_t i = next_.fetch_add(1);
            if (i >= job_n_) break;
            (*job_)(i);
        }
    }
    void loop_()
    {
        std::size_t seen = 0;
        for (;;)
        {
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return gen_ != seen; });
                seen = gen_;
                if (stop_) return;
            }
            run_();
            {
                std::lock_guard<std::mutex> lk(mu_);
                if (--pending_ == 0) done_cv_.notify_one();
            }
        }
    }

    std::vector<std::thread> workers_;
    std::mutex mu_, call_mu_;
    std::condition_variable cv_, done_cv_;
    const std::function<void(std::size_t)>* job_ = nullptr;
    std::size_t job_n_ = 0;
    std::atomic<std::size_t> next_{0};
    std::size_t pending_ = 0;
    std::size_t gen_ = 0;
    bool stop_ = false;
};

// Thread count: NNORACLE_THREADS if set, else hardware_concurrency (the
// reference's choice, core_threadpool.hpp:612).
inline std::size_t oracle_thread_count()
{
    if (const char* s = std::getenv("NNORACLE_THREADS"))
    {
        const long v = std::atol(s);
        if (v > 0) return static_cast<std::size_t>(v);
    }
    const unsigned hc = std::thread::hardware_concurrency();
    return hc == 0 ? 1 : hc;
}

inline ThreadPool& pool()
{
    static ThreadPool p(oracle_thread_count());
    return p;
}

// Elementwise helper: serial below the threshold, chunked-parallel above.
template <class F>
void for_range(std::size_t n, F&& f)
{
    if (n < PARALLEL_THRESHOLD)
    {
        for (std::size_t i = 0; i < n; ++i) f(i);
        return;
    }
    const std::size_t chunks = pool().size() * 4;
    const std::size_t step = (n + chunks - 1) / chunks;
    pool().parallel_for(chunks, [&](std::size_t c) {
        const std::size_t b = c * step, e = std::min(n, b + step);
        for (std::size_t i = b; i < e; ++i) f(i);
    });
}

inline float dot8_(const float* a, const float* b, std::size_t n)
{
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    std::size_t k = 0;
    for (; k + 8 <= n; k += 8)
        for (int l = 0; l < 8; ++l) acc[l] += a[k + l] * b[k + l];
    for (int l = 0; k < n; ++k, ++l) acc[l] += a[k] * b[k];
    return ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
}

// C (M,N) = op(A) op(B), C zero-initialised here. a_rows/a_cols and
// b_rows/b_cols are the stored shapes. transA: A stored (K,M); transB: B stored (N,K).
inline void gemm(float* C, std::size_t M, std::size_t N, std::size_t K, const float* A, std::size_t lda,
                 bool transA, const float* B, std::size_t ldb, bool transB)
{
    std::fill(C, C + M * N, 0.0f);
    if (M == 0 || N == 0 || K == 0) return;
    const std::size_t ib = (M + BLOCK - 1) / BLOCK, jb = (N + BLOCK - 1) / BLOCK;
    auto task = [&](std::size_t t) {
        const std::size_t i0 = (t / jb) * BLOCK, i1 = std::min(i0 + BLOCK, M);
        const std::size_t j0 = (t % jb) * BLOCK, j1 = std::min(j0 + BLOCK, N);
        std::array<float, BLOCK * BLOCK> bt{}, at{};
        for (std::size_t k0 = 0; k0 < K; k0 += BLOCK)
        {
            const std::size_t kl = std::min(BLOCK, K - k0);
            for (std::size_t j = j0; j < j1; ++j)
                for (std::size_t kk = 0; kk < kl; ++kk)
                    bt[(j - j0) * kl + kk] = transB ? B[j * ldb + k0 + kk] : B[(k0 + kk) * ldb + j];
            if (transA)
                for (std::size_t i = i0; i < i1; ++i)
                    for (std::size_t kk = 0; kk < kl; ++kk)
                        at[(i - i0) * kl + kk] = A[(k0 + kk) * lda + i];
            for (std::size_t i = i0; i < i1; ++i)
            {
                const float* arow = transA ? &at[(i - i0) * kl] : &A[i * lda + k0];
                float* crow = C + i * N;
                for (std::size_t j = j0; j < j1; ++j)
                    crow[j] += dot8_(arow, &bt[(j - j0) * kl], kl);
            }
        }
    };
    const std::size_t n = ib * jb;
    if (n <= 1) task(0);
    else pool().parallel_for(n, task);
}

inline void transpose(const float* src, float* dst, std::size_t R, std::size_t C)
{
    if (R == 0 || C == 0) return;
    const std::size_t ib = (R + BLOCK - 1) / BLOCK, jb = (C + BLOCK - 1) / BLOCK;
    auto task = [&](std::size_t t) {
        const std::size_t i0 = (t / jb) * BLOCK, i1 = std::min(i0 + BLOCK, R);
        const std::size_t j0 = (t % jb) * BLOCK, j1 = std::min(j0 + BLOCK, C);
        for (std::size_t i = i0; i < i1; ++i)
            for (std::size_t j = j0; j < j1; ++j) dst[j * R + i] = src[i * C + j];
    };
    if (ib * jb <= 1) task(0);
    else pool().parallel_for(ib * jb, task);
}

// Row reduction: out[r] = fold(init, A[r][0..C)) serially along the row.
template <class F>
void row_reduce(const float* A, float* out, std::size_t R, std::size_t C, float init, F&& f)
{
    auto row = [&](std::size_t r) {
        float acc = init;
        for (std::size_t c = 0; c < C; ++c) acc = f(acc, A[r * C + c]);
        out[r] = acc;
    };
    if (R >= PARALLEL_THRESHOLD) for_range(R, row);
    else for (std::size_t r = 0; r < R; ++r) row(r);
}

// Column reduction: serial row-major scan, or (R >= 1024 and R*C >= threshold)
// per-thread row-block partials combined in block order.
template <class F>
void col_reduce(const float* A, float* out, std::size_t R, std::size_t C, float init, F&& f)
{
    if (C == 0) return;
    const std::size_t nt = pool().size();
    if (R * C < 64 || R < 1024 || R * C < PARALLEL_THRESHOLD || nt <= 1)
    {
        for (std::size_t c = 0; c < C; ++c) out[c] = init;
        for (std::size_t r = 0; r < R; ++r)
            for (std::size_t c = 0; c < C; ++c) out[c] = f(out[c], A[r * C + c]);
        return;
    }
    std::vector<float> part(nt * C, init);
    const std::size_t base = R / nt, rem = R % nt;
    pool().parallel_for(nt, [&](std::size_t t) {
        const std::size_t r0 = t * base + std::min(t, rem), r1 = r0 + base + (t < rem ? 1 : 0);
        float* p = &part[t * C];
        for (std::size_t r = r0; r < r1; ++r)
            for (std::size_t c = 0; c < C; ++c) p[c] = f(p[c], A[r * C + c]);
    });
    for (std::size_t c = 0; c < C; ++c)
    {
        float acc = init;
        for (std::size_t t = 0; t < nt; ++t) acc = f(acc, part[t * C + c]);
        out[c] = acc;
    }
}

} // namespace nn::oracle
