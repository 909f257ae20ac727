// hip_engine.hpp — nn::ComputeEngine on one MI355X (gfx950) GPU.
//
// Drop-in replacement for the reference's GPU engines (GpuEngine, Vulkan,
// include/neuralnet.cpp/gpu_engine.hpp:49-961; CudaEngine,
// include/neuralnet.cpp/cuda_engine.hpp) behind the unchanged ComputeEngine
// interface. Every primitive validates shapes on the host exactly as the
// CPU engine does, allocates its outputs from a per-engine caching pool and
// enqueues hand-written HIP kernels (include/nnhip_kernels.h) on the engine's
// own stream. Nothing falls back to the CPU: an unsupported shape is an Error.
//
// Ordering: all work goes to one in-order stream, so a buffer released by a
// Tensor can be handed to the next allocation immediately (stream-ordered
// reuse). to_matrix and end_batch synchronise the stream, matching the
// reference's batch semantics (compute_engine.hpp:93-118); flush_batch
// submits the recorded work without waiting for it;
// from_matrix / copy_from copy small host data into a pinned staging slot and
// return once the upload is queued (larger data is uploaded and waited for).
//
// Deferred attention chains: the reference's two-pass attention calls
// (compute_layer.hpp:1196-1221, :1304-1327) are recorded instead of launched
// when their operands fit the one-pass kernels, and the whole chain runs as
// one launch when its last call arrives (reduce -> denom -> apply forward;
// batched_matmul(transA) -> backward_q -> backward_kv backward). The tensors a
// deferred call returns are real allocations; any other primitive that reads
// one of them, or writes in place to any tensor a deferred call uses, first
// launches the deferred work with the general kernels, and end_batch /
// flush_batch / settle() launch whatever is still deferred. A deferred result
// that nobody references any more is dropped without being computed.
//
// Deferred elementwise runs: consecutive in-place (add / scale / axpy) and
// elementwise (unary / binary / scalar / clone) calls on tensors of one size
// are recorded too, and run when any other call arrives (or on settle,
// end_batch, flush_batch, to_matrix). The optimizers' per-tensor Adam / AdamW
// chain (compute_optimizer.hpp:252-304, :388-412) is recognised among them and
// runs as one pass over p, m, v and g with the same roundings as the separate
// calls; everything else runs call by call.
#pragma once

#include <memory>
#include <optional>
#include <string>
#include <unordered_set>
#include <vector>

#include "compute_engine.hpp"

namespace nn
{

class DevicePool;
struct RunStep;

class HipEngine final : public ComputeEngine
{
public:
    // Engine on the current HIP device. Check ok() / error() after construction.
    HipEngine();
    ~HipEngine() override;
    HipEngine(const HipEngine&) = delete;
    HipEngine& operator=(const HipEngine&) = delete;

    [[nodiscard]] bool ok() const noexcept { return ok_; }
    [[nodiscard]] const std::string& error() const noexcept { return init_error_; }
    [[nodiscard]] void* stream() const noexcept { return stream_; }

    Device device() const noexcept override { return Device::GPU; }
    Result<void> begin_batch() override;
    Result<void> end_batch() override;
    Result<void> flush_batch() override;
    Result<void> begin_expr() override { return {}; }
    Result<void> end_expr() override { return {}; }

    Tensor create_tensor(std::size_t rows, std::size_t cols) override;
    Result<Tensor> from_matrix(const Matrix& m) override;
    Result<Matrix> to_matrix(const Tensor& t) override;
    Result<void> copy_from(Tensor& dst, const Matrix& src) override;
    Result<Tensor> clone(const Tensor& src) override;

    Result<Tensor> slice_rows(const Tensor& src, std::size_t start_row, std::size_t count) override;
    Result<void> insert_rows(Tensor& dst, std::size_t dst_start_row, const Tensor& src) override;
    Result<Tensor> gather_rows(const Tensor& table, const Tensor& indices) override;
    Result<void> scatter_add_rows(Tensor& dst, const Tensor& indices, const Tensor& grad) override;
    Result<Tensor> rearrange_3d(const Tensor& x, std::size_t M, std::size_t B, std::size_t N, bool inverse) override;
    Result<Tensor> transpose(const Tensor& A) override;

    Result<Tensor> matmul(const Tensor& A, const Tensor& B, bool transA, bool transB) override;
    Result<Tensor> batched_matmul(const Tensor& A, const Tensor& B, std::size_t batch, bool transA, bool transB,
                                  Scalar alpha) override;
    Result<Tensor> batched_matmul_reduce(const Tensor& A, const Tensor& B, std::size_t batch, ReduceOp op,
                                         bool transA, bool transB, Scalar alpha, bool reduce_cols,
                                         const Tensor* mask) override;
    Result<Tensor> batched_matmul_softmax_denom(const Tensor& A, const Tensor& B, const Tensor& row_max,
                                                std::size_t batch, bool transA, bool transB, Scalar alpha,
                                                const Tensor* mask) override;
    Result<Tensor> batched_matmul_softmax_apply(const Tensor& A, const Tensor& B, const Tensor& V,
                                                const Tensor& row_max, const Tensor& denom, std::size_t batch,
                                                bool transA, bool transB, Scalar alpha, const Tensor* mask) override;
    Result<Tensor> batched_matmul_softmax_backward_q(const Tensor& A, const Tensor& B, const Tensor& P,
                                                     const Tensor& row_max, const Tensor& denom, std::size_t batch,
                                                     bool transA, bool transB, Scalar alpha, Tensor& r_out,
                                                     const Tensor* mask) override;
    Result<Tensor> batched_matmul_softmax_backward_kv(const Tensor& A, const Tensor& B, const Tensor& P,
                                                      const Tensor& G, const Tensor& R, const Tensor& row_max,
                                                      const Tensor& denom, std::size_t batch, bool transA,
                                                      bool transB, Scalar alpha, Tensor& grad_v_out,
                                                      const Tensor* mask) override;

    Result<Tensor> col_softmax_denom(const Tensor& logits, const Tensor& col_max) override;
    Result<Tensor> col_softmax_sparse_forward(const Tensor& logits, const Tensor& labels, const Tensor* mask,
                                              std::size_t vocab_size, Scalar inv_num_valid,
                                              Tensor& loss_vec_out) override;

    Result<void> add_inplace(Tensor& A, const Tensor& B) override;
    Result<void> scale_inplace(Tensor& A, Scalar s) override;
    Result<void> axpy_inplace(Tensor& A, Scalar scalar, const Tensor& B) override;
    Result<void> zero(Tensor& A) override;

    Result<Tensor> row_reduce_sum(const Tensor& A) override;
    Result<Tensor> col_reduce_sum(const Tensor& A) override;
    Result<Tensor> row_reduce_max(const Tensor& A) override;
    Result<Tensor> col_reduce_max(const Tensor& A) override;

    Result<void> broadcast_row_inplace(Tensor& A, const Tensor& row_vec, BinaryOp op) override;
    Result<void> broadcast_col_inplace(Tensor& A, const Tensor& col_vec, BinaryOp op) override;

    Result<Tensor> elementwise_unary(UnaryOp op, const Tensor& A) override;
    Result<Tensor> elementwise_binary(BinaryOp op, const Tensor& A, const Tensor& B) override;
    Result<Tensor> elementwise_binary_scalar(BinaryOp op, const Tensor& A, Scalar s, bool scalar_first) override;
    Result<Tensor> elementwise_select_scalar_cond(CompareOp cmp, const Tensor& A, Scalar scalar_b,
                                                  const Tensor& then_t, Scalar scalar_else) override;

    Result<Tensor> eval_expr(const ExprSpec& spec, std::span<const Tensor> inputs, std::size_t rows,
                             std::size_t cols) override;
    Result<Tensor> eval_expr_reduce(const ExprSpec& spec, std::span<const Tensor> inputs, std::size_t rows,
                                    std::size_t cols) override;

    // Launches every deferred call whose results are still referenced (no wait).
    Result<void> settle();
    // Queues everything t's values depend on, as a read through the engine
    // would (the deferred producers, and for an attention probability tensor
    // that holds the forward's score blocks, the probabilities), without
    // waiting: t's memory holds its values once the stream reaches this point.
    Result<void> settle_for_read(const Tensor& t) override;

    // Bytes currently cached (free) and held by live tensors in the pool.
    [[nodiscard]] std::size_t pool_cached_bytes() const;
    [[nodiscard]] std::size_t pool_live_bytes() const;

    // Measurement hook: while enabled, every GEMM launch (matmul and
    // batched_matmul) is bracketed by HIP events on the engine's stream.
    // read_gemm_profile() waits for the stream and returns the number of
    // launches, their algorithmic FLOPs (2*M*N*K per batch) and the summed
    // kernel time in milliseconds, then clears the record.
    void set_gemm_profile(bool on);
    Result<void> read_gemm_profile(double& launches, double& flops, double& ms);
    // Same, plus one record per launch: {M, N, K, batch, transA, transB, ms}.
    Result<void> read_gemm_profile_records(std::vector<double>& records);

    // Bytes of attention score blocks that the two-pass chain's recorded
    // forward outputs may hold for their backward (default: 1/8 of the device
    // memory free at start-up, at most 8 GiB). 0 keeps none: every backward
    // then forms its scores again.
    void set_score_budget(std::size_t bytes) noexcept { score_budget_ = bytes; }

private:
    Result<Tensor> alloc_(std::size_t rows, std::size_t cols);
    // Row slices are views of their source's memory until the view or the
    // memory it aliases is written in place; then the view takes a private
    // copy first (copy semantics as CpuEngine, without copying slices that
    // are only read, e.g. SwiGLU's gate and up halves).
    Result<void> unshare_(const Tensor& t);
    Result<std::shared_ptr<DeviceBuffer>> scratch_(std::size_t bytes);
    Result<void> kernel_(int rc, const char* what);
    // Checks that every tensor lives on this engine, then launches deferred
    // work whose results are among them (the caller is about to read them).
    Result<void> need_gpu_(std::initializer_list<const Tensor*> ts, const char* what);
    Result<void> check_gpu_(std::initializer_list<const Tensor*> ts, const char* what) const;
    Result<void> sync_();   // waits for the stream (no deferred work is launched)
    Result<void> launch_gemm_(const Tensor& A, const Tensor& B, Tensor& C, std::size_t batch, bool tA, bool tB,
                              Scalar alpha, std::size_t M, std::size_t N, std::size_t K);

    // Mask cell tables of the one-pass attention kernels, kept per mask tensor
    // (most recent last) until the mask is written in place or evicted.
    struct OrderTable
    {
        std::size_t batch, N;
        int kind;
        bool per_batch;
        std::shared_ptr<DeviceBuffer> buf;
    };
    struct CellTable
    {
        Tensor mask;
        std::shared_ptr<DeviceBuffer> cells;
        std::size_t M;   // rows of one mask (the tensor holds rows / M of them)
        std::vector<OrderTable> orders;   // work orders of the launches over this table
    };
    std::vector<CellTable> cells_;
    // Work orders of multi-row launches, keyed by the rows' cell tables (kept
    // alive here, so a key never names a reused buffer), most recent last.
    struct RowsOrder
    {
        std::vector<std::shared_ptr<DeviceBuffer>> cells;
        std::size_t hpr, M, N;
        int kind;
        std::shared_ptr<DeviceBuffer> buf;
    };
    std::vector<RowsOrder> rows_orders_;
    Result<std::shared_ptr<DeviceBuffer>> mask_cells_buf_(const Tensor* mask, std::size_t M, std::size_t N);
    Result<const void*> rows_order_(const std::vector<std::shared_ptr<DeviceBuffer>>& cells, std::size_t hpr,
                                    std::size_t M, std::size_t N, int kind);
    // Fused two-pass attention launches (softmax_apply's forward; backward_kv's
    // backward from the forward's output) recorded instead of launched. On
    // demand all of them run: the forwards first, then the backwards, calls of
    // one kind and shape (e.g. the packed rows of a document-masked batch, one
    // call per row) together as multi-row launches.
    struct PendingFlash;
    std::vector<PendingFlash> pflash_;
    bool flash_yields_(const float* p) const;
    bool flash_uses_(const float* p) const;
    Result<void> settle_flash_();
    Result<void> launch_flash_(const std::vector<const PendingFlash*>& rows);
    std::size_t score_budget_ = 0;
    std::vector<std::weak_ptr<DeviceBuffer>> views_;   // live row-slice views (HipView)
    // Every live aliased view and its root (may also hold buffers no longer
    // in that role): a write to any other buffer needs no unsharing.
    std::unordered_set<const DeviceBuffer*> view_keys_;
    Result<const void*> mask_cells_(const Tensor* mask, std::size_t M, std::size_t N);
    Result<const void*> flash_order_(const void* cells, std::size_t batch, std::size_t M, std::size_t N,
                                     std::size_t mask_bs, int kind);

    struct PendingFwd;
    struct PendingGemm;
    struct PendingBwd;
    struct PendingEw;
    struct PendingSwb;
    std::vector<PendingSwb> pswb_;
    Result<void> settle_swb_();
    struct PendingMm;
    std::unique_ptr<PendingMm> pmm_;
    // Earlier matmuls still recorded when the next one did not read them
    // (the attention's q, k, v projections), oldest first.
    std::vector<std::unique_ptr<PendingMm>> pmm_prev_;
    Result<void> settle_mm_();
    Result<void> settle_mm_prev_(const float* p, bool write);
    Result<void> launch_pending_mm_(std::unique_ptr<PendingMm> o);
    Result<void> launch_mm_(const PendingMm& r, const Tensor& out, const Tensor* bias, bool accumulate);
    PendingMm* pending_mm_(const Tensor& t);
    PendingMm* vec_record_(const Tensor& t);
    PendingMm* vec_slice_of_(const Tensor& t, std::size_t& off);
    struct PendingAcc;
    std::unique_ptr<PendingAcc> pacc_;
    Result<void> settle_acc_();
    struct PendingMaskAdd;
    struct PendingAttn;
    struct PendingDv;
    struct PendingDs;
    struct AttnGrads;
    std::unique_ptr<PendingMaskAdd> pmadd_;
    std::vector<std::shared_ptr<PendingAttn>> pattn_;   // one per layer between forward and backward
    std::unique_ptr<PendingDv> pdv_;
    std::unique_ptr<PendingDs> pds_;
    std::unique_ptr<AttnGrads> pgrads_;
    Result<void> settle_madd_();
    Result<void> settle_dv_();
    Result<void> settle_ds_();
    Result<void> materialise_attn_(PendingAttn& p);
    Result<std::optional<Tensor>> attn_query_(PendingAttn& p, const Tensor& V, std::size_t Dv);
    void forget_dead_attn_();
    std::shared_ptr<PendingAttn> attn_of_(const Tensor& A) const;
    Result<void> scores_masked_(const Tensor& Q, const Tensor& K, const Tensor& mask, std::size_t batch, std::size_t M,
                                std::size_t N, std::size_t Kd, float alpha, const Tensor& out);
    Result<std::optional<Tensor>> attn_bmm_(const Tensor& A, const Tensor& B, std::size_t batch, bool tA, bool tB,
                                            Scalar alpha);
    Result<std::optional<Tensor>> attn_softmax_(const ExprSpec& spec, std::span<const Tensor> inputs,
                                                std::size_t rows, std::size_t cols);
    // transpose calls (and rearrange_3d of them) not launched yet, most recent last.
    struct PendingLayout;
    std::vector<PendingLayout> playout_;
    Result<void> push_layout_(PendingLayout r);
    Result<void> materialise_layout_(const PendingLayout& r);
    Result<void> settle_layout_();
    const PendingLayout* layout_of_(const Tensor& t) const;
    const PendingLayout* merge_of_(const Tensor& t) const;
    Result<void> settle_layout_for_(const Tensor& t);
    // A row sum not launched yet (a Linear bias gradient, RMSNorm's gamma gradient).
    struct PendingRowSum;
    std::unique_ptr<PendingRowSum> prsum_;
    Result<void> settle_rsum_();
    Result<void> launch_rsum_(const PendingRowSum& r, float* out, bool add);
    // RMSNorm::forward's calls from the sum of squares on, not launched yet.
    struct PendingRms;
    std::unique_ptr<PendingRms> prms_;
    Result<void> settle_rms_();
    Result<std::optional<Tensor>> rms_program_(const ExprSpec& spec, std::span<const Tensor> inputs,
                                               std::size_t rows, std::size_t cols, bool vector_out);
    // Outputs of the two-pass chain's forward kept for the backward, one per layer.
    struct TwoPassOut;
    std::vector<TwoPassOut> ptwo_;
    void forget_dead_two_();
    std::unique_ptr<PendingFwd> pfwd_;
    std::unique_ptr<PendingGemm> pgemm_;
    std::unique_ptr<PendingBwd> pbwd_;
    std::unique_ptr<PendingEw> pew_;
    struct PendingZero
    {
        Tensor t;
        std::vector<std::pair<std::size_t, std::size_t>> covered;   // rows inserted since the zero call
    };
    // zero calls not yet launched; each is launched when its memory is first
    // read or written (or on settle), so zero_grad's fills wait for the
    // backward, whose first accumulation into a gradient becomes a write.
    std::vector<PendingZero> pzero_;
    Result<void> settle_zero_();
    Result<void> settle_zero_for_(const Tensor& t);
    bool take_zero_(const Tensor& t);
    Result<void> zero_now_(const Tensor& t);
    Result<void> launch_zero_(std::vector<PendingZero>& ts);
    // Before reading (writing) tensors: launch deferred work that yields
    // (yields or reads) them; the plain forms also launch the elementwise run.
    Result<void> settle_reads_(std::initializer_list<const Tensor*> ts);
    Result<void> settle_write_(const Tensor& t);
    // keep_flash: recorded fused attention launches stay recorded even if they
    // yield one of the tensors (the caller records work that runs after them).
    Result<void> settle_chain_reads_(std::initializer_list<const Tensor*> ts, bool keep_flash = false);
    // keep_swb: placed SwiGLU records stay; keep_zero: t's own zero record stays
    Result<void> settle_chain_write_(const Tensor& t, bool keep_swb = false, bool keep_zero = false);
    Result<void> ew_push_(unsigned code, unsigned op, bool first, const Tensor& dst, const Tensor& a, const Tensor* b,
                          float s);
    // keep_adam: recognised Adam chains stay collected in padam_ (the record
    // is being replaced by one of another size; the next call is recorded too).
    Result<void> settle_ew_(bool keep_adam = false);
    // Adam / AdamW update chains recognised in elementwise records and not yet
    // launched: launched together (nnhip_adam_update_list) before any other
    // kernel, so their order relative to every other call is kept.
    struct PendingAdam
    {
        Tensor p, m, v, g;
    };
    std::vector<PendingAdam> padam_;
    float padam_args_[11] = {};   // has_decay, decay, beta1, 1-beta1, beta2, 1-beta2, ib1, ib2, eps, -lr, (unused)
    Result<void> flush_adam_();
    Result<std::size_t> adam_run_(const PendingEw& g, std::size_t i, const std::vector<std::ptrdiff_t>& last_read);
    Result<std::size_t> swiglu_run_(const PendingEw& g, std::size_t i, const std::vector<std::ptrdiff_t>& last_read);
    Result<std::size_t> swiglu_vec_run_(const PendingEw& g, const std::vector<std::ptrdiff_t>& last_read);
    static bool match_run_(const PendingEw& g, std::size_t i, const RunStep* steps, std::size_t len, int nroles,
                           int* slot_of);
    Result<void> settle_fwd_();
    Result<void> settle_gemm_();
    Result<void> settle_bwd_();
    Result<std::shared_ptr<DeviceBuffer>> attn_ws_(std::size_t batch, std::size_t M, std::size_t N, std::size_t K,
                                                   std::size_t D);
    std::optional<Result<Tensor>> fused_layer_program_(const ExprSpec& spec, std::span<const Tensor> inputs,
                                                       std::size_t rows, std::size_t cols, bool vector_out);
    Result<Tensor> eval_impl_(const ExprSpec& spec, std::span<const Tensor> inputs, std::size_t rows,
                              std::size_t cols, bool vector_out);

    void prof_begin_();
    void prof_end_(std::size_t M, std::size_t N, std::size_t K, std::size_t batch, bool tA, bool tB);

    struct ProfRecord
    {
        void* start;
        void* stop;
        double flops;
        double shape[6];   // M, N, K, batch, transA, transB
    };
    bool profile_ = false;
    std::vector<ProfRecord> prof_;
    std::vector<void*> event_pool_;

    // Pinned staging ring for small uploads (from_matrix, copy_from): the
    // call returns once its upload is queued. Returns false (nothing done)
    // when the data does not fit a slot.
    Result<bool> upload_(float* dst, const float* src, std::size_t n);
    static constexpr std::size_t kStageSlot = std::size_t(256) << 10, kStageSlots = 64;
    void* stage_ = nullptr;
    std::vector<void*> stage_ev_;
    std::size_t stage_next_ = 0;

    bool ok_ = false;
    std::string init_error_;
    int device_ = 0;
    void* stream_ = nullptr;
    std::shared_ptr<DevicePool> pool_;
};

} // namespace nn
