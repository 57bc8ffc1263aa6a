// Host-side constants and helpers shared by the C-ABI entry points of libgpic_fp8.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gpic_fp8.h"

namespace gpic {

constexpr int kCastThreads = 256;                     // threads per workgroup of the streaming cast kernels
constexpr int kMaxParts = 1024;                       // at most this many partial maxima per amax pass
constexpr int kMaxCastBlocks = 8192;                  // workgroups of a streaming cast pass
constexpr size_t kCastWorkspaceBytes = kMaxParts * 4; // the partial maxima

static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace gpic
