// Words of the data-polled exchanges (a consumer polls the data itself until no
// word reads the empty marker the buffer was filled with).  Plain C++ so that
// the host test suite compiles it with g++ and checks it exhaustively.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define MKD_HD __host__ __device__ __forceinline__
#else
#define MKD_HD inline
#endif

namespace mkd {

// Empty marker of a bf16 exchange buffer: the 16-bit word 0xffff (a negative
// NaN with a full payload).
constexpr uint32_t kPollEmptyBf16 = 0xffffu;
// The quiet NaN a producer stores instead of a value whose bf16 bits equal the
// marker, so that a NaN result stays a NaN and the consumer's poll still ends.
constexpr uint32_t kPollNanBf16 = 0x7fc0u;

// A packed bf16 pair as a producer stores it into a bf16 exchange buffer: each
// half equal to the empty marker becomes the quiet NaN, every other pattern is
// kept bit for bit.
MKD_HD uint32_t poll_safe_bf16x2(uint32_t p) {
  const uint32_t lo = (p & 0xffffu) == kPollEmptyBf16 ? kPollNanBf16 : (p & 0xffffu);
  const uint32_t hi = (p >> 16) == kPollEmptyBf16 ? kPollNanBf16 : (p >> 16);
  return lo | (hi << 16);
}

// A consumer's test of one 32-bit word of a bf16 exchange buffer: true while
// either half still holds the marker.
MKD_HD bool poll_bf16x2_empty(uint32_t v) {
  return (v & 0xffffu) == kPollEmptyBf16 || (v >> 16) == kPollEmptyBf16;
}

}  // namespace mkd
