// Decode-step glue kernels: embedding gather, greedy arg-max, RoPE tables.
#include "common.h"
#include "mkd_internal.h"

namespace mkd {

__global__ void embed_kernel(const int* __restrict__ ids, const uint16_t* __restrict__ table,
                             uint16_t* __restrict__ out, int H, int V) {
  const int b = blockIdx.y;
  const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i >= H) return;
  const int id = ids[b];
  // an out-of-vocabulary id yields a zero row instead of a read outside the table
  const u32x4_t z = {0, 0, 0, 0};
  st16(out + (long long)b * H + i, (id >= 0 && id < V) ? ld16(table + (long long)id * H + i) : z);
}

// Stage 1: each block reduces a slice of one row to (max, first index).
// Stage 2 (last block per row, by atomic ticket): reduces the block results.
constexpr int kArgThreads = 256;
constexpr int kArgBlocks = 64;

MKD_DEV void argbest(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i) || (v != v && v2 == v2)) { v = v2; i = i2; }
}

__global__ void __launch_bounds__(kArgThreads)
argmax_kernel(const float* __restrict__ logits, int V, int* __restrict__ out,
              float* __restrict__ sv, int* __restrict__ si) {
  const int b = blockIdx.y;
  const float* row = logits + (long long)b * V;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int j = blockIdx.x * kArgThreads + threadIdx.x; j < V; j += kArgBlocks * kArgThreads)
    argbest(bv, bi, row[j], j);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(bv, o, 64);
    const int i2 = __shfl_xor(bi, o, 64);
    argbest(bv, bi, v2, i2);
  }
  __shared__ float wv[kArgThreads / 64];
  __shared__ int wi[kArgThreads / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) { wv[w] = bv; wi[w] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int q = 1; q < kArgThreads / 64; ++q) argbest(bv, bi, wv[q], wi[q]);
    sv[b * kArgBlocks + blockIdx.x] = bv;
    si[b * kArgBlocks + blockIdx.x] = bi;
  }
}

__global__ void argmax_final_kernel(const float* __restrict__ sv, const int* __restrict__ si,
                                    int* __restrict__ out) {
  const int b = blockIdx.x;
  float bv = sv[b * kArgBlocks + threadIdx.x];
  int bi = si[b * kArgBlocks + threadIdx.x];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(bv, o, 64);
    const int i2 = __shfl_xor(bi, o, 64);
    argbest(bv, bi, v2, i2);
  }
  if (threadIdx.x == 0) out[b] = bi;
}

// cos/sin [B, d] fp32 with duplicated halves: angle = pos * inv_freq[i mod d/2].
__global__ void rope_table_kernel(const int* __restrict__ pos, const float* __restrict__ inv_freq,
                                  int d, float* __restrict__ cosv, float* __restrict__ sinv) {
  const int b = blockIdx.x, i = threadIdx.x;
  const float ang = (float)pos[b] * inv_freq[i % (d / 2)];
  cosv[b * d + i] = cosf(ang);
  sinv[b * d + i] = sinf(ang);
}

hipError_t embed_launch(const int* ids, const uint16_t* table, uint16_t* out, int B, int H, int V,
                        hipStream_t s) {
  if (H % 8) return hipErrorInvalidValue;
  hipLaunchKernelGGL(embed_kernel, dim3((H / 8 + 255) / 256, B), dim3(256), 0, s, ids, table, out, H, V);
  return hipGetLastError();
}

hipError_t argmax_launch(const float* logits, int B, int V, int* out, float* scratch_val,
                         int* scratch_idx, hipStream_t s) {
  hipLaunchKernelGGL(argmax_kernel, dim3(kArgBlocks, B), dim3(kArgThreads), 0, s, logits, V, out,
                     scratch_val, scratch_idx);
  hipLaunchKernelGGL(argmax_final_kernel, dim3(B), dim3(kArgBlocks), 0, s, scratch_val,
                     scratch_idx, out);
  return hipGetLastError();
}

hipError_t rope_table_launch(const int* pos, const float* inv_freq, int B, int d, float* cos,
                             float* sin, hipStream_t s) {
  hipLaunchKernelGGL(rope_table_kernel, dim3(B), dim3(d), 0, s, pos, inv_freq, d, cos, sin);
  return hipGetLastError();
}

}  // namespace mkd
