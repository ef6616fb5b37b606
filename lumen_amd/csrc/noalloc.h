// Limits and scratch of lumen_sampler_sample_batch_noalloc (noalloc.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace lumen {

constexpr uint32_t kNoAllocMaxRows = 8;          // rows per call
constexpr uint32_t kNoAllocMaxVocab = 262144;    // logits per row
constexpr uint32_t kNoAllocMaxCsr = 65536;       // form-A penalty entries per call
constexpr size_t kNoAllocBytes = (size_t)32 << 20;  // the device array, per GPU

hipError_t noalloc_scratch(void** out);

}  // namespace lumen
