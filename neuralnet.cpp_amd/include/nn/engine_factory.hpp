// engine_factory.hpp — engine selection with the reference's rules
// (include/neuralnet.cpp/cli/engine_factory.hpp:45-88), with HIP added.
//
// Priority HIP > CUDA > Vulkan > CPU. A backend that is requested and cannot
// be created is an error, never a silent fall back to another engine; the
// caller decides whether to stop. This library holds the HIP engine only:
// CUDA and Vulkan requests name the reference's own engines, and with no
// request the reference returns its CpuEngine, which lives in the
// reference, so here that case is an error that says so.
#pragma once

#include <memory>
#include <ostream>
#include <string>

#include "compute_engine.hpp"
#include "core_errors.hpp"
#include "hip_engine.hpp"

namespace nn::cli
{

struct EngineConfig
{
    bool use_gpu = false;    // Vulkan GpuEngine (reference)
    bool use_cuda = false;   // CudaEngine (reference)
    bool use_hip = false;    // HipEngine (this library); first in priority
};

[[nodiscard]] inline Result<std::unique_ptr<ComputeEngine>> create_engine(const EngineConfig& cfg, std::ostream* log)
{
    if (cfg.use_hip)
    {
        auto e = std::make_unique<HipEngine>();
        if (!e->ok())
            return fail("--hip requested but HIP initialisation failed: " + e->error() +
                        " (no fallback to another engine)");
        if (log) *log << "HIP GPU engine enabled (HipEngine, gfx950)\n";
        return std::unique_ptr<ComputeEngine>(std::move(e));
    }
    if (cfg.use_cuda)
        return fail("--cuda requested: this library has no CUDA engine (the reference's CudaEngine); no fallback");
    if (cfg.use_gpu)
        return fail("--gpu requested: this library has no Vulkan engine (the reference's GpuEngine); no fallback");
    return fail("no engine requested: this library provides the HIP engine only (request use_hip); the CPU engine "
                "is the reference's CpuEngine");
}

} // namespace nn::cli
