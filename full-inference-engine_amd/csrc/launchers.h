// Host-side launchers of the large kernels, one translation unit each
// (k_scan.hip, k_finish_*.hip, k_lmhead.hip), so the library builds in parallel.
// Each returns the launch's hipError_t; the C ABI in sampler.hip reports it.
#pragma once

#include "scan.h"

namespace fie {

constexpr int kLhKAlign = 128;   // the fused lm_head's hidden size must be a multiple

// k_scan over grid (spans, rows).
hipError_t launch_scan(const KParams& P, bool vec, bool longh, hipStream_t st);

// k_finish (one workgroup per row; `wide` = the 256-register variant that settles
// full-row rows itself), or k_deep over the queued rows when `deep`.
hipError_t launch_finish_f32(const KParams& P, bool vec, bool deep, bool wide, hipStream_t st);
hipError_t launch_finish_f16(const KParams& P, bool vec, bool deep, bool wide, hipStream_t st);
hipError_t launch_finish_bf16(const KParams& P, bool vec, bool deep, bool wide, hipStream_t st);

// k_lmhead (fp16 / bf16 only).
hipError_t launch_lmhead(const KParams& P, const void* hidden, const void* weight, int H, bool vec,
                         bool longh, hipStream_t st);

}  // namespace fie
