// Host-side constants and helpers shared by the C-ABI entry points of libgpic_fp8.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gpic_fp8.h"

namespace gpic {

constexpr int kCastThreads = 256;                     // threads per workgroup of the streaming cast kernels
constexpr int kMaxParts = 1024;                       // at most this many partial maxima per amax pass
constexpr int kAmaxBlocks = 512;                      // workgroups of a flat amax pass
constexpr int kSwigluBlocks = 512;                    // workgroups of a SwiGLU pass
constexpr int kMaxCastBlocks = 8192;                  // workgroups of a streaming cast pass
constexpr int kCastTBlocks = 1024;                    // workgroups of a (persistent) transposing cast pass
constexpr int kSwigluCastTBlocks = 768;               // workgroups of the SwiGLU backward's recomputing cast (3 per CU)
constexpr size_t kCastWorkspaceBytes = 40 * 1024;     // partial maxima (4 KiB), the SwiGLU sigmoid table (24 KiB),
                                                      // the single-pass tagged partials (8 KiB) and call counter

static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace gpic
