// Shared device helpers for the gfx950 kernels: bf16 storage, wave64
// reductions, Philox4x32-10, status reporting.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>
#include <string>
#include "../../include/flaxchat_amd.h"

typedef uint16_t bf16_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// bf16 MFMA 32x32x16 (gfx950): lane l holds row / column l % 32 and k values
// 8 (l / 32) .. +7 of each operand; the result register 4 i + x of lane l is
// row 8 i + 4 (l / 32) + x, column l % 32.
__device__ __forceinline__ f32x16 mfma32(v4u a, v4u b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                  0, 0);
}

#define WAVE 64

__device__ __forceinline__ float bf2f(bf16_t h) { return __uint_as_float(((uint32_t)h) << 16); }
__device__ __forceinline__ bf16_t f2bf(float f) {
  // round to nearest even (inputs here are finite)
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
}

// Fragment order of a bf16 matrix-core operand [R][K] (R padded to a
// multiple of 16, K a multiple of 32): 16-row x 32-k blocks of 1 KB in
// [row block][k step] order; inside a block, the 16 bytes at offset 16 l
// are row l % 16, k = 8 (l / 16) .. +7 of the step, which is exactly what
// lane l of a 16x16x32 MFMA takes as its operand. One wave-wide 16-byte load
// then reads 1 KB contiguous. Weights and the bf16 GEMM activations are
// stored this way; fp32 (parity mode) operands stay row-major.
__host__ __device__ __forceinline__ int64_t frag_idx(int64_t r, int k, int K) {
  return ((((r >> 4) * (K >> 5) + (k >> 5)) << 9) | ((int64_t)((r & 15) | (((k & 31) >> 3) << 4)) << 3) |
          (k & 7));
}
template <typename T> __device__ __forceinline__ int64_t act_idx(int64_t r, int k, int K);
template <> __device__ __forceinline__ int64_t act_idx<uint16_t>(int64_t r, int k, int K) { return frag_idx(r, k, K); }
template <> __device__ __forceinline__ int64_t act_idx<float>(int64_t r, int k, int K) { return r * K + k; }
__host__ __device__ __forceinline__ int64_t round16(int64_t r) { return (r + 15) / 16 * 16; }

// K cache of the matrix-core path (bf16, head_dim 128): 32-key blocks of
// 8 KB in the fragment order of the S^T = K Q^T product. In a block, load
// (cc, s) of lane l = r + 16 g (1 KB contiguous) holds key
// 8 (r / 4) + r % 4 + 4 cc, dims 32 s + 8 g .. +7; so element (key kk of
// the block, dim d) sits at ((2 s + cc) 64 + r + 16 g) 8 + d % 8 with
// s = d / 32, g = (d / 8) % 4, r = 4 (kk / 8) + kk % 4, cc = (kk / 4) % 2.
__device__ __forceinline__ int64_t kblk_idx(int pos, int d) {
  const int kk = pos & 31;
  const int r = ((kk >> 3) << 2) | (kk & 3), cc = (kk >> 2) & 1;
  const int s = d >> 5, g = (d >> 3) & 3;
  return (int64_t)(pos >> 5) * 4096 + ((((s << 1) | cc) << 6) + r + (g << 4)) * 8 + (d & 7);
}

// Packed tokens of row b (row_off as in fc_chunk): n = 0 when the descriptor
// is out of range (more than max_per_row tokens, or past the capacity), so a
// bad descriptor feeds nothing instead of addressing outside the buffers.
struct RowSpan {
  int base, n;
};
__device__ __forceinline__ RowSpan row_span(const int* row_off, int b, int max_per_row, int Mcap) {
  const int base = row_off[b], n = row_off[b + 1] - base;
  if (base < 0 || n <= 0 || n > max_per_row || base + n > Mcap) return RowSpan{0, 0};
  return RowSpan{base, n};
}

template <typename T> __device__ __forceinline__ float ld(const T* p, int64_t i);
template <> __device__ __forceinline__ float ld<float>(const float* p, int64_t i) { return p[i]; }
template <> __device__ __forceinline__ float ld<bf16_t>(const bf16_t* p, int64_t i) { return bf2f(p[i]); }
template <typename T> __device__ __forceinline__ void st(T* p, int64_t i, float v);
template <> __device__ __forceinline__ void st<float>(float* p, int64_t i, float v) { p[i] = v; }
template <> __device__ __forceinline__ void st<bf16_t>(bf16_t* p, int64_t i, float v) { p[i] = f2bf(v); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
  return v;
}
// (value, index) argmax: larger value wins, lower index among equals.
__device__ __forceinline__ void argmax_merge(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float v2 = __shfl_xor(v, o, WAVE);
    int i2 = __shfl_xor(i, o, WAVE);
    argmax_merge(v, i, v2, i2);
  }
}

// Block reductions through a small LDS buffer (>= 16 floats). All threads
// receive the result.
__device__ __forceinline__ float block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}
__device__ __forceinline__ float block_max(float v, float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int i = 0; i < nw; ++i) t = fmaxf(t, red[i]);
  return t;
}
__device__ __forceinline__ void block_argmax(float& v, int& idx, float* redv, int* redi) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  wave_argmax(v, idx);
  __syncthreads();
  if (lane == 0) { redv[w] = v; redi[w] = idx; }
  __syncthreads();
  float bv = redv[0];
  int bi = redi[0];
  for (int i = 1; i < nw; ++i) argmax_merge(bv, bi, redv[i], redi[i]);
  v = bv;
  idx = bi;
}

// ---------------------------------------------------------------------------
// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11). Counter (c0..c3), key
// (k0, k1); 10 rounds, key bumped by the Weyl constants between rounds.
// ---------------------------------------------------------------------------
struct u32x4 { uint32_t x, y, z, w; };
__device__ __forceinline__ u32x4 philox4x32_10(u32x4 c, uint32_t k0, uint32_t k1) {
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) { k0 += W0; k1 += W1; }
    const uint32_t lo0 = M0 * c.x, hi0 = __umulhi(M0, c.x);
    const uint32_t lo1 = M1 * c.z, hi1 = __umulhi(M1, c.z);
    c = u32x4{hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0};
  }
  return c;
}
__device__ __forceinline__ uint32_t pick(const u32x4& r, int i) {
  return i == 0 ? r.x : (i == 1 ? r.y : (i == 2 ? r.z : r.w));
}
// u in (0, 1) for Gumbel noise: 23 random bits plus one half, exact in fp32
// (with 24 bits, (2^24 - 1) + 0.5 rounds to 2^24 and u would reach 1.0);
// u in [0, 1) for accept tests.
__device__ __forceinline__ float u_open(uint32_t bits) { return ((float)(bits >> 9) + 0.5f) * 1.1920928955078125e-7f; }
__device__ __forceinline__ float u_half(uint32_t bits) { return (float)(bits >> 8) * 5.9604644775390625e-8f; }
// standard Gumbel noise -log(-log(u)) of one Philox word
__device__ __forceinline__ float gumbel_of(uint32_t bits) { return -logf(-logf(u_open(bits))); }

// ---------------------------------------------------------------------------
// Host-side status plumbing
// ---------------------------------------------------------------------------
void fc_set_error(const std::string& s);
#define FC_CHECK_ARG(cond, msg)                 \
  do {                                          \
    if (!(cond)) {                              \
      fc_set_error(std::string("argument: ") + msg); \
      return FC_ERR_ARG;                        \
    }                                           \
  } while (0)
#define FC_HIP(call)                                                         \
  do {                                                                       \
    hipError_t e_ = (call);                                                  \
    if (e_ != hipSuccess) {                                                  \
      fc_set_error(std::string(#call) + ": " + hipGetErrorString(e_));       \
      return FC_ERR_HIP;                                                     \
    }                                                                        \
  } while (0)
#define FC_LAUNCH_CHECK()                                                    \
  do {                                                                       \
    hipError_t e_ = hipGetLastError();                                       \
    if (e_ != hipSuccess) {                                                  \
      fc_set_error(std::string("launch: ") + hipGetErrorString(e_));         \
      return FC_ERR_HIP;                                                     \
    }                                                                        \
  } while (0)

static inline int64_t fc_align(int64_t x, int64_t a = 256) { return (x + a - 1) / a * a; }
