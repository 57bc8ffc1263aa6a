// The single-pass fold shared by the kernels that reduce a tensor to its maximum and cast it in one launch (the
// flat and transposing casts, the normalisation that casts its output): every workgroup publishes a partial maximum
// in the cast workspace and takes the maximum of all of them, with bounded waits.
#pragma once
#include "gpic_device.h"
#include "gpic_launch.h"

namespace gpic {

// Partials: one 64-bit word per workgroup, (call tag << 32) | amax bits, in the workspace. The tag is the workspace's
// epoch + 1 (0 skipped): thread 0 of every workgroup reads the epoch as the kernel starts (once_epoch, its latency
// hidden behind the kernel's first loads) and, once it has the value, counts its workgroup done; the last workgroup of
// the call to be counted (a counter in the workspace reaching the grid size) stores the tag as the new epoch at its end
// (once_done) and clears the counter. So the epoch cannot change before every workgroup of the call has read it, and
// the next call on the workspace -- stream-ordered after this one, or the next replay of a captured graph -- uses the
// next tag: a word left by an earlier call never matches, and a word this call's waiters publish late carries this
// call's tag, which the next call does not use. The workspace is zeroed once, when it is created, and tag 0 is never
// used; the tag repeats after 2^32 calls on one workspace.
// No workgroup waits on another without a bound: a partial that has not appeared within the wait bound (kOnceWaitUs by
// default, about 8x a whole call) is computed by the waiting workgroup itself, from that workgroup's share of x, and
// published for the other waiters. So the launch needs no co-residency guarantee (a plain launch; the cooperative one
// costs ~17 us per call here), never deadlocks when other work holds CUs, and the amax is exact either way. The
// workspace's fallback word counts such direct computations (0 in normal runs).
// A single-pass kernel calls once_epoch before its first loads, once_fold once, and once_done as its last statement
// (every thread reaches it). The done counts are issued in once_fold and their results looked at only later, so their
// round trips pass while the workgroup waits for the other partials and casts, instead of delaying the casts.
constexpr int kMaxOnceBlocks = 1024;
constexpr size_t kOnceTagged = 28 * 1024;                         // uint64_t[kMaxOnceBlocks] tagged partials
constexpr size_t kOnceFallback = kOnceTagged + 8 * kMaxOnceBlocks;  // uint32_t: partials computed by a waiter
constexpr size_t kOnceEpoch = kOnceFallback + 4;                    // uint32_t: the tag of the last call
constexpr size_t kOnceDone = kOnceFallback + 8;                     // uint32_t: groups of this call done folding
// Per group of kDoneGroup workgroups, the count of its workgroups done folding, each on its own 128-byte line: a single
// counter taking one atomic from each of 1024 workgroups measured ~10 us per call (they serialise on one address).
constexpr int kDoneGroup = 32;
constexpr size_t kOnceGroupDone = 40 * 1024;                        // uint32_t at kOnceGroupDone + 128 g
static_assert(kOnceDone + 4 <= kOnceGroupDone, "single-pass words overlap");
static_assert(kOnceGroupDone + 128 * ((kMaxOnceBlocks + kDoneGroup - 1) / kDoneGroup) <= kCastWorkspaceBytes,
              "cast workspace too small");
constexpr int kOnceWaitUs = 200;   // the default bound of a wait for another workgroup's partial (about 8x a cast)

// The call's tag, kept in LDS between once_fold and once_done.
__device__ __forceinline__ uint32_t &once_tag_slot() {
  __shared__ uint32_t tag;
  return tag;
}
// The epoch, read by thread 0 (the other threads return 0). Relaxed atomics throughout: the epoch is written only by
// the previous call's last workgroup, which ended before this kernel started, and an acquire / release at agent scope
// would write back or invalidate whole caches on this multi-XCD part in each of the 1024 workgroups.
__device__ __forceinline__ uint32_t once_epoch(void *ws) {
  return threadIdx.x == 0 ? __hip_atomic_load(reinterpret_cast<uint32_t *>((char *)ws + kOnceEpoch), __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT)
                          : 0u;
}
// Publishes this workgroup's maximum m (held by every thread) as this call's partial, then returns the maximum over
// all G partials to every thread. epoch: once_epoch's value (used by thread 0). share_max(c) must return (to every
// thread of the workgroup) workgroup c's maximum computed from x; it runs only for a partial that did not appear within
// wait_ticks. ticket: for once_done (thread 0's count of groups done, or ~0 where this workgroup completes no group).
// The done count has two levels: the last workgroup of each group of kDoneGroup counts its group done (atomic
// read-modify-writes of one address are totally ordered, so exactly one workgroup sees each count complete); every
// counter is back at zero when the call ends.
// once_fold_range: the same over the partials of workgroups [first, first + count) only (a launch that casts several
// tensors, each over its own range of workgroups); share_max then takes the index within the range.
template <class ShareMax>
__device__ __forceinline__ uint32_t once_fold_range(uint32_t m, void *ws, uint32_t epoch, uint32_t wait_ticks,
                                                    uint32_t &ticket, int first, int count, ShareMax share_max) {
  __shared__ int missing[kMaxOnceBlocks];
  __shared__ int nmissing;
  uint32_t &stag = once_tag_slot();
  uint64_t *tagged = reinterpret_cast<uint64_t *>((char *)ws + kOnceTagged);
  const int G = gridDim.x;
  const int grp = blockIdx.x / kDoneGroup;
  uint32_t *gdone = reinterpret_cast<uint32_t *>((char *)ws + kOnceGroupDone + 128 * grp);
  uint32_t gticket = 0;
  if (threadIdx.x == 0) {
    uint32_t t = epoch + 1u;
    t = t ? t : 1u;
    stag = t;
    __hip_atomic_store(tagged + blockIdx.x, ((uint64_t)t << 32) | m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    nmissing = 0;
    // Counted done: issued after the tag (so after the epoch load has returned: the tag's stores wait for it), its
    // result looked at only after the partials have been read. (The compiler does not move atomics past each other.)
    asm volatile("" ::: "memory");
    gticket = __hip_atomic_fetch_add(gdone, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const uint32_t tag = stag;
  uint32_t g = m;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (int i = first + (int)threadIdx.x; i < first + count; i += blockDim.x) {
    uint64_t w = __hip_atomic_load(tagged + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    while ((uint32_t)(w >> 32) != tag && __builtin_amdgcn_s_memrealtime() - t0 < wait_ticks) {
      __builtin_amdgcn_s_sleep(2);
      w = __hip_atomic_load(tagged + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if ((uint32_t)(w >> 32) == tag) g = max(g, (uint32_t)w);
    else missing[atomicAdd(&nmissing, 1)] = i;
  }
  g = block_max_u32(g);   // its barriers also publish `missing`
  const int nm = nmissing;
  if (nm > 0) {
    // Waiters help each other: each starts at a different missing partial, computes it from x and publishes it (the
    // same word its owner writes), and checks every other one again before computing it, so the missing partials are
    // computed about once between all waiters rather than once by each.
    __shared__ uint64_t seen;
    int computed = 0;
    for (int k = 0; k < nm; k++) {
      const int c = missing[(k + blockIdx.x) % nm];
      if (threadIdx.x == 0)   // (a zero wait bound skips the check: every partial missing at the first poll is computed)
        seen = wait_ticks ? __hip_atomic_load(tagged + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
      __syncthreads();
      const uint64_t w = seen;
      __syncthreads();   // `seen` is rewritten by the next iteration
      if ((uint32_t)(w >> 32) == tag) {
        g = max(g, (uint32_t)w);
      } else {
        const uint32_t v = share_max(c - first);
        g = max(g, v);
        computed++;
        if (threadIdx.x == 0)
          __hip_atomic_store(tagged + c, ((uint64_t)tag << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (threadIdx.x == 0 && computed > 0)
      __hip_atomic_fetch_add(reinterpret_cast<uint32_t *>((char *)ws + kOnceFallback), (uint32_t)computed,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  ticket = ~0u;
  if (threadIdx.x == 0 && gticket == (uint32_t)min(kDoneGroup, G - grp * kDoneGroup) - 1u) {   // this group is done
    __hip_atomic_store(gdone, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ticket = __hip_atomic_fetch_add(reinterpret_cast<uint32_t *>((char *)ws + kOnceDone), 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
  }
  return g;
}
template <class ShareMax>
__device__ __forceinline__ uint32_t once_fold(uint32_t m, void *ws, uint32_t epoch, uint32_t wait_ticks,
                                              uint32_t &ticket, ShareMax share_max) {
  return once_fold_range(m, ws, epoch, wait_ticks, ticket, 0, (int)gridDim.x, share_max);
}
// The last statement of a single-pass kernel (ticket: once_fold's): the workgroup that completed the last group
// clears the count and stores the call's tag as the new epoch.
__device__ __forceinline__ void once_done(void *ws, uint32_t ticket) {
  if (threadIdx.x == 0 && ticket == (uint32_t)((gridDim.x + kDoneGroup - 1) / kDoneGroup) - 1u) {
    __hip_atomic_store(reinterpret_cast<uint32_t *>((char *)ws + kOnceDone), 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(reinterpret_cast<uint32_t *>((char *)ws + kOnceEpoch), once_tag_slot(), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Host side (cast.hip): workgroups of `kernel` (`threads` threads each) the current device holds at once, capped at
// kMaxOnceBlocks and cached per device in `cache`; the wait bound in s_memrealtime ticks; whether single-pass
// launches are enabled (gpic_fp8_set_single_pass).
int once_capacity(const void *kernel, DeviceCache &cache, int threads);
uint32_t once_wait_ticks();
bool once_enabled();

}  // namespace gpic
