// Host-side declarations shared between the library's translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rtxllm {

// Greedy token kernels (decode_kernels.cu:2993-3073). mode 0: token =
// (argmax + token + 1) % 32000 (the decode chain); mode 1: token = (argmax +
// offset) % vocab. argmax keeps the lowest index among equal maxima.
hipError_t launch_argmax_token(const float* logits, std::uint32_t* token, std::uint32_t rows, int mode,
                               std::uint32_t vocab, std::uint32_t offset, hipStream_t stream);

}  // namespace rtxllm
