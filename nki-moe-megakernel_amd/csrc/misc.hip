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

__global__ void decode_begin_kernel(DecodeBeginArgs d) {
  const long long tid = blockIdx.x * (long long)blockDim.x + threadIdx.x;
  const long long nth = (long long)gridDim.x * blockDim.x;
  if (d.cos)
    for (long long i = tid; i < (long long)d.B * d.d; i += nth) {
      const int b = (int)(i / d.d), k = (int)(i % d.d);
      const float ang = (float)d.pos[b] * d.inv_freq[k % (d.d / 2)];
      d.cos[i] = cosf(ang);
      d.sin[i] = sinf(ang);
    }
  for (long long i = tid; i < d.sync_words; i += nth) d.sync[i] = 0u;
  if (!d.poll) return;
  // chunks the attention can read: those holding positions 0 .. n (the prior
  // rows and the new token), n the position clamped like the prior length
  const int n = min(max(d.pos[0], 0), d.S_max);
  const int nch = min((n + 1 + d.chunk - 1) / d.chunk, d.n_chunks);
  // per layer: one run of nch * D words per head (chunk partials), one of
  // nch * 2 per head (their max / sum), and the whole tail; one block per run
  // at a time, 16-byte stores where the run starts 16-byte aligned
  const long long tail = d.layer_words - d.po - d.pml;
  const long long runs = 2LL * d.nq + 1;
  for (long long ru = blockIdx.x; ru < runs * d.layers; ru += gridDim.x) {
    const long long l = ru / runs;
    const int j = (int)(ru % runs);
    long long off, len;
    if (j < d.nq) {
      off = (long long)j * d.n_chunks * d.D;
      len = (long long)nch * d.D;
    } else if (j < 2 * d.nq) {
      off = d.po + (long long)(j - d.nq) * d.n_chunks * 2;
      len = 2LL * nch;
    } else {
      off = d.po + d.pml;
      len = tail;
    }
    uint32_t* p = d.poll + l * d.layer_words + off;
    long long done = 0;
    if ((reinterpret_cast<uintptr_t>(p) & 15) == 0) {
      const long long n4 = len / 4;
      for (long long i = threadIdx.x; i < n4; i += blockDim.x)
        reinterpret_cast<u32x4_t*>(p)[i] = u32x4_t{kPollEmpty, kPollEmpty, kPollEmpty, kPollEmpty};
      done = n4 * 4;
    }
    for (long long i = done + threadIdx.x; i < len; i += blockDim.x) p[i] = kPollEmpty;
  }
}

hipError_t decode_begin_launch(const DecodeBeginArgs& d, hipStream_t s) {
  long long work = d.cos ? (long long)d.B * d.d : 0;
  work = max(work, (long long)d.sync_words);
  if (d.poll) {
    if (d.B != 1 || d.chunk <= 0 || d.n_chunks <= 0 || d.po != (long long)d.nq * d.n_chunks * d.D ||
        d.pml != (long long)d.nq * d.n_chunks * 2 || d.layer_words < d.po + d.pml)
      return hipErrorInvalidValue;
    work = max(work, d.layer_words * d.layers);
  }
  if (work <= 0) return hipSuccess;
  const long long blocks = min((work + 255) / 256, 1024LL);
  hipLaunchKernelGGL(decode_begin_kernel, dim3((unsigned)blocks), dim3(256), 0, s, d);
  return hipGetLastError();
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
