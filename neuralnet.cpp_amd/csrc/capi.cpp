// capi.cpp — the engine C-ABI (include/nnhip_engine.h) over HipEngine.
#include <iostream>

#include "nn/engine_capi.hpp"
#include "nn/engine_factory.hpp"
#include "nn/hip_engine.hpp"

namespace
{
std::unique_ptr<nn::ComputeEngine> make_hip_engine(std::string& err)
{
    auto e = std::make_unique<nn::HipEngine>();
    if (!e->ok())
    {
        err = e->error();
        return nullptr;
    }
    return e;
}
} // namespace

NN_DEFINE_ENGINE_CAPI(nnhip_, make_hip_engine(err))

// Measurement hooks (no reference counterpart): GEMM kernel time by HIP events.
extern "C" NN_CAPI_EXPORT int nnhip_engine_profile_gemm(void* e, int enable)
{
    auto* h = dynamic_cast<nn::HipEngine*>(static_cast<nn::capi::EngineHandle*>(e)->eng.get());
    if (!h) return nn::capi::set_error("profile: not a HIP engine");
    h->set_gemm_profile(enable != 0);
    return 0;
}

extern "C" NN_CAPI_EXPORT int nnhip_engine_profile_gemm_read(void* e, double* launches, double* flops, double* ms)
{
    auto* h = dynamic_cast<nn::HipEngine*>(static_cast<nn::capi::EngineHandle*>(e)->eng.get());
    if (!h) return nn::capi::set_error("profile: not a HIP engine");
    auto r = h->read_gemm_profile(*launches, *flops, *ms);
    return r ? 0 : nn::capi::set_error(r.error().message);
}

// Per-launch records {M, N, K, batch, transA, transB, ms} of the profiled GEMMs
// (7 doubles each); returns the number of records, at most `max`, or -1.
extern "C" NN_CAPI_EXPORT long nnhip_engine_profile_gemm_records(void* e, double* out, size_t max)
{
    auto* h = dynamic_cast<nn::HipEngine*>(static_cast<nn::capi::EngineHandle*>(e)->eng.get());
    if (!h) return nn::capi::set_error("profile: not a HIP engine"), -1;
    std::vector<double> rec;
    auto r = h->read_gemm_profile_records(rec);
    if (!r) return nn::capi::set_error(r.error().message), -1;
    const size_t n = std::min(rec.size() / 7, max);
    std::copy(rec.begin(), rec.begin() + static_cast<std::ptrdiff_t>(7 * n), out);
    return static_cast<long>(n);
}

extern "C" NN_CAPI_EXPORT void* nnhip_engine_stream(void* e)
{
    auto* h = dynamic_cast<nn::HipEngine*>(static_cast<nn::capi::EngineHandle*>(e)->eng.get());
    return h ? h->stream() : nullptr;
}

// Launches every deferred attention call whose results are still referenced,
// without waiting (HipEngine::settle); end_batch does the same and then waits.
extern "C" NN_CAPI_EXPORT int nnhip_engine_settle(void* e)
{
    auto* h = dynamic_cast<nn::HipEngine*>(static_cast<nn::capi::EngineHandle*>(e)->eng.get());
    if (!h) return nn::capi::set_error("settle: not a HIP engine");
    auto r = h->settle();
    return r ? 0 : nn::capi::set_error(r.error().message);
}

// Bytes of attention score blocks the two-pass chain's recorded forwards may
// keep for their backward (HipEngine::set_score_budget).
extern "C" NN_CAPI_EXPORT int nnhip_engine_set_score_budget(void* e, size_t bytes)
{
    auto* h = dynamic_cast<nn::HipEngine*>(static_cast<nn::capi::EngineHandle*>(e)->eng.get());
    if (!h) return nn::capi::set_error("set_score_budget: not a HIP engine");
    h->set_score_budget(bytes);
    return 0;
}

// cli::create_engine with the reference's flags (cli/engine_factory.hpp:45-88)
// plus use_hip: the requested backend or an error, never another engine.
extern "C" NN_CAPI_EXPORT int nnhip_engine_select(int use_hip, int use_cuda, int use_gpu, int verbose, void** out)
{
    if (!out) return nn::capi::set_error("engine_select: null output");
    *out = nullptr;
    nn::cli::EngineConfig cfg;
    cfg.use_hip = use_hip != 0;
    cfg.use_cuda = use_cuda != 0;
    cfg.use_gpu = use_gpu != 0;
    auto r = nn::cli::create_engine(cfg, verbose ? &std::cerr : nullptr);
    if (!r) return nn::capi::set_error(r.error().message);
    *out = new nn::capi::EngineHandle{std::move(*r)};
    return 0;
}
