// ORACLE — test infrastructure only (loaded by tests/, __graft_entry__.smoke()
// and bench.py's cpu_baseline leg, never by the product).
//
// Exports the engine C-ABI of include/nnhip_engine.h with the prefix
// `nnoracle_` over the CpuEngine restatement, so tests drive the CPU oracle
// and the HIP engine through identical calls.
#include "cpu_engine.hpp"
#include "nn/engine_capi.hpp"

NN_DEFINE_ENGINE_CAPI(nnoracle_, std::unique_ptr<nn::ComputeEngine>(new nn::oracle::CpuEngine()))

extern "C" NN_CAPI_EXPORT size_t nnoracle_thread_count(void) { return nn::oracle::pool().size(); }
