// model_spec.hpp — architecture enums of the GPT path.
//
// Numeric values are those of include/neuralnet.cpp/model_spec.hpp:24-47
// (they are stored in the reference's model files).
#pragma once

#include <cstdint>

namespace nn
{

enum class PosEncodingType : std::uint32_t { Learned = 0, Sinusoidal = 1, ALiBi = 2, RoPE = 3 };
enum class ActivationType : std::uint32_t { GeLU = 0, SwiGLU = 1 };
enum class NormType : std::uint32_t { LayerNorm = 0, RMSNorm = 1, BatchNorm = 2 };

} // namespace nn
