// Skinny GEMMs with fused epilogues: out = epi(A[M][K] . W[N][K]^T).
//
// Replaces the nnx.Linear matmuls of the per-token forward
// (flaxchat/engine.py:106-108, 158, 161, 172; flaxchat/gpt.py:93-99, 154-163)
// and fuses what the reference does right after them: the residual add
// (engine.py:160-161), ReLU^2 (gpt.py:161), resid/x0 lambda mix of the next
// layer (engine.py:94), the backout capture and subtraction
// (engine.py:164-166) and the 15*tanh(z/15) softcap (engine.py:173-174).
//
// Three kernels, chosen by M (= rows = batch x tokens per row):
//   k_gemv      VALU dot products; fp32 weights (parity mode) or bf16 with
//               M < 16, where a 16-row matrix-core tile would be mostly empty.
//   k_gemm_sk   bf16 MFMA 16x16x32, 16 output columns per workgroup, the
//               four waves split K and reduce through LDS (M <= 64).
//   k_gemm_wide bf16 MFMA, 64 columns per workgroup, the A tile staged in
//               LDS and shared by the four waves (M > 64).
// Weights stream from HBM exactly once per M tile; each lane loads 16 bytes
// per row segment so a wave reads 64 contiguous bytes of each of 16 rows.
#include "fc_common.h"
#include "fc_internal.h"

__device__ __forceinline__ void epi_apply(const Epi& e, int m, int n, float acc) {
  switch (e.mode) {
    case EPI_STORE: {
      ((float*)e.out)[(int64_t)m * e.ldo + n] = acc;
      break;
    }
    case EPI_ADD: {
      float* o = (float*)e.out + (int64_t)m * e.ldo + n;
      *o = *o + acc;
      break;
    }
    case EPI_RELU2: {
      float r = fmaxf(acc, 0.f);
      r = r * r;
      if (e.out_dtype == FC_BF16) ((bf16_t*)e.out)[(int64_t)m * e.ldo + n] = f2bf(r);
      else ((float*)e.out)[(int64_t)m * e.ldo + n] = r;
      break;
    }
    case EPI_MLPOUT: {
      const int64_t i = (int64_t)m * e.ldo + n;
      float* x = (float*)e.out;
      const float t = x[i] + acc;             // x + mlp(...)        engine.py:161
      float xb_v = 0.f;
      if (e.capture) { e.xb[i] = t; xb_v = t; } // x_backout          engine.py:164
      else if (e.last) xb_v = e.xb[i];
      if (e.last) x[i] = t - e.lb * xb_v;       // x - lambda * x_b    engine.py:166
      else x[i] = e.r * t + e.a * e.x0[i];      // next layer's mix    engine.py:94
      break;
    }
    case EPI_SOFTCAP: {
      if (n < e.V) {
        const int b = m / e.n_out, rr = m - b * e.n_out;
        ((float*)e.out)[(int64_t)b * e.row_stride + (int64_t)rr * e.V + n] = 15.f * tanhf(acc / 15.f);
      }
      break;
    }
  }
}

// ---------------------------------------------------------------------------
// VALU GEMV / small GEMM. 256 threads = 4 waves; each wave owns 4 columns
// and MB rows; lanes split K in 16-byte vectors.
// ---------------------------------------------------------------------------
template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const T* p, float* o);
template <>
__device__ __forceinline__ void load_vec<float, 4>(const float* p, float* o) {
  float4 v = *(const float4*)p;
  o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
}
template <>
__device__ __forceinline__ void load_vec<float, 8>(const float* p, float* o) {
  load_vec<float, 4>(p, o);
  load_vec<float, 4>(p + 4, o + 4);
}
template <>
__device__ __forceinline__ void load_vec<bf16_t, 8>(const bf16_t* p, float* o) {
  uint4 v = *(const uint4*)p;
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __uint_as_float(w[i] << 16);
    o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void load_vec<bf16_t, 4>(const bf16_t* p, float* o) {
  uint2 v = *(const uint2*)p;
  o[0] = __uint_as_float(v.x << 16);
  o[1] = __uint_as_float(v.x & 0xffff0000u);
  o[2] = __uint_as_float(v.y << 16);
  o[3] = __uint_as_float(v.y & 0xffff0000u);
}

template <typename T, int MB>
__global__ __launch_bounds__(256) void k_gemv(const T* __restrict__ A, const T* __restrict__ W,
                                              int M, int N, int K, Epi e) {
  constexpr int VEC = 16 / sizeof(T);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wave) * 4;
  const int m0 = blockIdx.y * MB;
  float acc[MB][4];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[i][c] = 0.f;
  for (int k = lane * VEC; k < K; k += 64 * VEC) {
    float w[4][VEC];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (n0 + c < N) load_vec<T, VEC>(W + (int64_t)(n0 + c) * K + k, w[c]);
      else
#pragma unroll
        for (int j = 0; j < VEC; ++j) w[c][j] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      if (m0 + i < M) {
        float a[VEC];
        load_vec<T, VEC>(A + (int64_t)(m0 + i) * K + k, a);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int j = 0; j < VEC; ++j) acc[i][c] += a[j] * w[c][j];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[i][c] = wave_sum(acc[i][c]);
  // spread the stores over lanes: lane (i*4 + c) stores element (i, c)
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (lane == ((i * 4 + c) & 63) && m0 + i < M && n0 + c < N) epi_apply(e, m0 + i, n0 + c, acc[i][c]);
}

// ---------------------------------------------------------------------------
// bf16 MFMA 16x16x32. Operand layout (wave64): lane l holds row (l % 16) of
// A / column (l % 16) of B and the 8 consecutive k values 8*(l/16)..+7 of a
// 32-wide k step; the f32x4 result holds rows 4*(l/16)+i of column l % 16.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ f32x4 mfma16(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

template <int MB>
__global__ __launch_bounds__(256) void k_gemm_sk(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W,
                                                 int M, int N, int K, Epi e) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int m0 = blockIdx.y * 16 * MB;
  f32x4 acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bf16_t* wrow = W + (int64_t)(n0 + r) * K + 8 * g;
  const uint4 zero = {0u, 0u, 0u, 0u};
  for (int kc = wave * 128; kc < K; kc += 512) {
    uint4 wf[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) wf[s] = *(const uint4*)(wrow + kc + 32 * s);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int am = m0 + 16 * mb + r;
      const bf16_t* arow = A + (int64_t)am * K + kc + 8 * g;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint4 af = am < M ? *(const uint4*)(arow + 32 * s) : zero;
        acc[mb] = mfma16(af, wf[s], acc[mb]);
      }
    }
  }
  __shared__ f32x4 red[3][MB][64];
  if (wave > 0)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) red[wave - 1][mb][lane] = acc[mb];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      f32x4 t = acc[mb];
#pragma unroll
      for (int w = 0; w < 3; ++w) t += red[w][mb][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * mb + 4 * g + i;
        if (m < M) epi_apply(e, m, n0 + r, t[i]);
      }
    }
  }
}

template <int MB>
__global__ __launch_bounds__(256) void k_gemm_wide(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W,
                                                   int M, int N, int K, Epi e) {
  constexpr int LDA = 128 + 8;  // bf16 elements per LDS row (padded)
  __shared__ bf16_t As[16 * MB * LDA];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 64 + wave * 16;
  const int m0 = blockIdx.y * 16 * MB;
  f32x4 acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bf16_t* wrow = W + (int64_t)(n0 + r) * K + 8 * g;
  const int srow = t >> 4, scol = (t & 15) * 8;
  const uint4 zero = {0u, 0u, 0u, 0u};
  for (int kc = 0; kc < K; kc += 128) {
    uint4 wf[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) wf[s] = *(const uint4*)(wrow + kc + 32 * s);
    uint4 stage[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const int gm = m0 + srow + 16 * i;
      stage[i] = gm < M ? *(const uint4*)(A + (int64_t)gm * K + kc + scol) : zero;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MB; ++i) *(uint4*)(As + (srow + 16 * i) * LDA + scol) = stage[i];
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const uint4 af = *(const uint4*)(As + (16 * mb + r) * LDA + 32 * s + 8 * g);
        acc[mb] = mfma16(af, wf[s], acc[mb]);
      }
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + 16 * mb + 4 * g + i;
      if (m < M) epi_apply(e, m, n0 + r, acc[mb][i]);
    }
}

// ---------------------------------------------------------------------------
// Dispatch
// ---------------------------------------------------------------------------
template <typename T>
static void launch_gemv(const void* A, const void* W, int M, int N, int K, const Epi& e, hipStream_t s) {
  dim3 blk(256);
  if (M <= 1) {
    hipLaunchKernelGGL((k_gemv<T, 1>), dim3((N + 15) / 16, M), blk, 0, s, (const T*)A, (const T*)W, M, N, K, e);
  } else if (M <= 2) {
    hipLaunchKernelGGL((k_gemv<T, 2>), dim3((N + 15) / 16, 1), blk, 0, s, (const T*)A, (const T*)W, M, N, K, e);
  } else if (M <= 4) {
    hipLaunchKernelGGL((k_gemv<T, 4>), dim3((N + 15) / 16, 1), blk, 0, s, (const T*)A, (const T*)W, M, N, K, e);
  } else {
    hipLaunchKernelGGL((k_gemv<T, 8>), dim3((N + 15) / 16, (M + 7) / 8), blk, 0, s, (const T*)A, (const T*)W, M, N,
                       K, e);
  }
}

int fc_launch_gemm(const void* A, const void* W, int M, int N, int K, int dtype, const Epi& e, hipStream_t s) {
  if (M <= 0 || N <= 0) return FC_OK;
  FC_CHECK_ARG(K > 0 && K % 8 == 0, "gemm K must be a positive multiple of 8");
  if (dtype == FC_F32) {
    launch_gemv<float>(A, W, M, N, K, e, s);
  } else if (M < 16 || K % 128 != 0 || N % 16 != 0) {
    launch_gemv<bf16_t>(A, W, M, N, K, e, s);
  } else if (M <= 64 || N % 64 != 0) {
    const int mb = (M + 15) / 16;
    if (mb <= 1)
      hipLaunchKernelGGL((k_gemm_sk<1>), dim3(N / 16, 1), dim3(256), 0, s, (const bf16_t*)A, (const bf16_t*)W, M, N,
                         K, e);
    else if (mb <= 2)
      hipLaunchKernelGGL((k_gemm_sk<2>), dim3(N / 16, 1), dim3(256), 0, s, (const bf16_t*)A, (const bf16_t*)W, M, N,
                         K, e);
    else
      hipLaunchKernelGGL((k_gemm_sk<4>), dim3(N / 16, (M + 63) / 64), dim3(256), 0, s, (const bf16_t*)A,
                         (const bf16_t*)W, M, N, K, e);
  } else {
    if (M <= 128)
      hipLaunchKernelGGL((k_gemm_wide<8>), dim3(N / 64, 1), dim3(256), 0, s, (const bf16_t*)A, (const bf16_t*)W, M,
                         N, K, e);
    else
      hipLaunchKernelGGL((k_gemm_wide<16>), dim3(N / 64, (M + 255) / 256), dim3(256), 0, s, (const bf16_t*)A,
                         (const bf16_t*)W, M, N, K, e);
  }
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int32_t fc_gemm(const void* A, const void* W, void* out, int32_t M, int32_t N, int32_t K, int32_t dtype,
                           int32_t epi, void* stream) {
  FC_CHECK_ARG(A && W && out, "null pointer");
  FC_CHECK_ARG(dtype == FC_F32 || dtype == FC_BF16, "dtype");
  FC_CHECK_ARG(epi == EPI_STORE || epi == EPI_ADD || epi == EPI_RELU2 || epi == EPI_SOFTCAP, "epilogue");
  Epi e{};
  e.mode = epi;
  e.out = out;
  e.ldo = N;
  e.out_dtype = dtype;
  e.n_out = 1;
  e.row_stride = N;
  e.V = N;
  return fc_launch_gemm(A, W, M, N, K, dtype, e, (hipStream_t)stream);
}
