// Device-coherent accesses for data exchanged between blocks of ONE launch.
//
// The per-XCD L2 caches of MI355X are not coherent with each other: a plain
// store sits in the writer's L2 and a plain load may hit a stale line in the
// reader's.  Stores and loads that carry the buffer cache-policy bit sc1 go to
// the device coherence point on both sides, so once a writer's sc1 stores have
// completed (s_waitcnt vmcnt(0)) and it has published a flag word (sc1 store),
// a reader that sees the flag (sc1 load) and then reads the data (sc1 loads)
// gets the new values -- no cache write-back or invalidate is needed.
#pragma once
#include "common.h"

namespace mkd {

constexpr int kCohSc1 = 16;                 // buffer cache-policy bit sc1
constexpr unsigned kCohSpinLimit = 1u << 20;

typedef unsigned coh_u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned coh_u32x4 __attribute__((ext_vector_type(4)));

MKD_DEV __amdgpu_buffer_rsrc_t coh_rsrc(const void* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, 0x7fffffff, 0x00020000);
}
MKD_DEV u32x4_t coh_ld16(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCohSc1));
}
MKD_DEV void coh_st8(__amdgpu_buffer_rsrc_t r, int off, uint32_t lo, uint32_t hi) {
  __builtin_amdgcn_raw_buffer_store_b64(coh_u32x2{lo, hi}, r, off, 0, kCohSc1);
}
MKD_DEV void coh_st16(__amdgpu_buffer_rsrc_t r, int off, u32x4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(coh_u32x4, v), r, off, 0, kCohSc1);
}
MKD_DEV void coh_st2(__amdgpu_buffer_rsrc_t r, int off, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, kCohSc1);
}
MKD_DEV unsigned coh_load(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
MKD_DEV void coh_store(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
MKD_DEV float coh_ldf(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
MKD_DEV void coh_stf(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
MKD_DEV uint32_t coh_ld4(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kCohSc1);
}
MKD_DEV coh_u32x2 coh_ld8(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kCohSc1);
}
MKD_DEV uint16_t coh_ld2(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, kCohSc1);
}
// vmcnt(0): every load and store this wave issued has completed
MKD_DEV void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0xF70); }

// Block barrier for LDS data only: this wave's LDS accesses have completed,
// then s_barrier.  Unlike __syncthreads (whose workgroup fence waits for every
// outstanding vector-memory access, vmcnt(0)) it leaves loads in flight -- the
// global -> LDS copies and the next round of polls.  A compiler barrier too.
MKD_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Publish a block's results: every wave waits for its own stores, then thread 0
// sets the block's flag word.  Called by all threads of the block.
MKD_DEV void coh_publish(unsigned* flag) {
  wait_vm_all();
  __syncthreads();
  if (threadIdx.x == 0) coh_store(flag, 1u);
}

// A data-polling loop's bound (same as coh_wait_all's): true once *err is set
// (another wait already gave up) or after kCohSpinLimit polls, when it sets
// *err itself; the caller then goes on with whatever it read.
MKD_DEV bool coh_poll_giveup(unsigned it, unsigned* err) {
  if (coh_load(err) != 0u) return true;
  if (it >= kCohSpinLimit) {
    if ((threadIdx.x & 63) == 0) coh_store(err, 1u);
    return true;
  }
  return false;
}

// One wave waits until the n flag words fl[0..n) are all non-zero.  Bounded:
// after kCohSpinLimit polls (tens of milliseconds) it sets *err and gives up, and
// a wave that finds *err already set does not wait at all, so the grid always
// drains (the results of such a launch are invalid; the host reads *err).
MKD_DEV void coh_wait_all(const unsigned* fl, int n, unsigned* err) {
  const int lane = threadIdx.x & 63;
  if (coh_load(err) != 0u) return;
  for (unsigned it = 0;; ++it) {
    bool ok = true;
    for (int c0 = 0; c0 < n; c0 += 64)
      ok &= (c0 + lane >= n) || coh_load(fl + c0 + lane) != 0u;
    if (__all(ok)) return;
    if (it >= kCohSpinLimit) {
      if (lane == 0) coh_store(err, 1u);
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

}  // namespace mkd
