// C++ drop-in for the reference's launch API, header-only over the C ABI of
// latent_attn.h (link with liblatent_attn_hip.so). Includes the three
// reference-shaped headers, whose names live in the global namespace like the
// reference's (paths relative to the reference repo):
//
//   mla_config.hpp         MLAConfig, LatentKVCache     src/mla_config.cuh:7-92
//   fused_mla.hpp          FusedMLAParams, launch_fused_mla
//                                                       src/fused_mla.cuh:11-51
//   fused_mla_batched.hpp  BatchedFusedMLAParams, launch_batched_fused_mla
//                                                       src/fused_mla_batched.cuh:7-35
//
// and repeats them in namespace latent_attn for callers that qualify them.
#pragma once

#include "fused_mla.hpp"
#include "fused_mla_batched.hpp"
#include "mla_config.hpp"

namespace latent_attn {
using ::BatchedFusedMLAParams;
using ::FusedMLAParams;
using ::LatentKVCache;
using ::MLAConfig;
using ::fused_mla_workspace_size;
using ::launch_batched_fused_mla;
using ::launch_fused_mla;
inline hipError_t to_hip_error(int status) { return ::la_to_hip_error(status); }
}  // namespace latent_attn
