// Skinny GEMMs with fused epilogues: out = epi(A[M][K] . W[N][K]^T).
//
// Replaces the nnx.Linear matmuls of the per-token forward
// (flaxchat/engine.py:106-108, 158, 161, 172; flaxchat/gpt.py:93-99, 154-163)
// and fuses what the reference does right after them: the residual add
// (engine.py:160-161), ReLU^2 (gpt.py:161), resid/x0 lambda mix of the next
// layer (engine.py:94), the backout capture and subtraction
// (engine.py:164-166) and the 15*tanh(z/15) softcap (engine.py:173-174).
//
// Kernels, chosen by M (= rows = batch x tokens per row):
//   k_gemv        VALU dot products; fp32 weights (parity mode) or bf16 with
//                 M < 16, where a 16-row matrix-core tile would be mostly empty.
//   k_gemm_stream bf16 MFMA 16x16x32 for M <= 64 (draft steps): pure weight
//                 streaming. A workgroup owns 16 output columns; its four
//                 waves split K and each wave issues the 16-byte weight loads
//                 of up to four 128-wide k chunks before the first MFMA, so
//                 ~16 KB per wave are in flight; the activation rows come
//                 straight from L2.
//   k_gemm_tile   bf16 MFMA for M > 64 (verify / prefill). A workgroup owns
//                 up to 256 rows x 128 columns; the activation chunk is staged
//                 in LDS (double buffered) and each wave reuses every A
//                 fragment for two 16-column blocks, halving LDS traffic per
//                 MFMA; weight fragments for the next chunk are prefetched.
// When N alone gives too few workgroups to occupy 256 CUs, a GEMM whose
// output is the fp32 residual stream may split K across workgroups: each
// split writes its partial product with plain stores and the RMSNorm kernel
// that consumes x next sums the splits in fixed order and applies the
// epilogue (a kernel boundary is the only synchronisation; on MI355X the
// eight XCD L2 caches are not coherent, so an in-kernel device-scope fence
// would write back a whole L2 per workgroup).
#include "fc_common.h"
#include "fc_internal.h"

template <int EPI>
__device__ __forceinline__ void epi_apply(const Epi e, int m, int n, float acc) {
  if constexpr (EPI == EPI_STORE) {
    ((float*)e.out)[(int64_t)m * e.ldo + n] = acc;
  } else if constexpr (EPI == EPI_ADD) {
    float* o = (float*)e.out + (int64_t)m * e.ldo + n;
    *o = *o + acc;
  } else if constexpr (EPI == EPI_RELU2) {
    float r = fmaxf(acc, 0.f);
    r = r * r;
    if (e.out_dtype == FC_BF16) ((bf16_t*)e.out)[(int64_t)m * e.ldo + n] = f2bf(r);
    else ((float*)e.out)[(int64_t)m * e.ldo + n] = r;
  } else if constexpr (EPI == EPI_MLPOUT) {
    const int64_t i = (int64_t)m * e.ldo + n;
    float* x = (float*)e.out;
    const float t = x[i] + acc;  // x + mlp(...)                 engine.py:161
    float xb_v = 0.f;
    if (e.capture) {             // x_backout                    engine.py:164
      e.xb[i] = t;
      xb_v = t;
    } else if (e.last) {
      xb_v = e.xb[i];
    }
    if (e.last) x[i] = t - e.lb * xb_v;      // x - lambda * x_b  engine.py:166
    else x[i] = e.r * t + e.a * e.x0[i];     // next layer's mix  engine.py:94
  } else if constexpr (EPI == EPI_PARTIAL) {  // split-K partial, finished by the next RMSNorm
    e.part[((int64_t)e.split * e.part_rows + m) * e.ldo + n] = acc;
  } else {                                   // EPI_SOFTCAP
    if (n < e.V) {
      const int b = m / e.n_out, rr = m - b * e.n_out;
      ((float*)e.out)[(int64_t)b * e.row_stride + (int64_t)rr * e.V + n] = 15.f * tanhf(acc / 15.f);
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
__device__ __forceinline__ void load_vec<bf16_t, 8>(const bf16_t* p, float* o) {
  uint4 v = *(const uint4*)p;
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __uint_as_float(w[i] << 16);
    o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

template <typename T, int MB, int EPI>
__global__ __launch_bounds__(256) void k_gemv(const T* __restrict__ A, const T* __restrict__ W, int M, int N,
                                              int K, Epi e) {
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
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (lane == ((i * 4 + c) & 63) && m0 + i < M && n0 + c < N) epi_apply<EPI>(e, m0 + i, n0 + c, acc[i][c]);
}

// ---------------------------------------------------------------------------
// bf16 MFMA 16x16x32. Operand layout (wave64): lane l holds row (l % 16) of
// A / column (l % 16) of B and 8 consecutive k values 8*(l/16)..+7 of a
// 32-wide k step; the f32x4 result holds rows 4*(l/16)+i of column l % 16.
// ---------------------------------------------------------------------------
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f32x4 mfma16(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                  0, 0);
}
__device__ __forceinline__ f32x4 mfma16(v4u a, v4u b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                  0, 0);
}

// M <= 64: streaming. grid (N/64, S, ceil(M/(16 MB))). A workgroup owns 64
// columns (4 N-blocks) so each activation fragment fetched from L2 feeds four
// MFMAs; its four waves split K in 128-wide chunks and each wave keeps two
// chunks of weight fragments (32 KB per wave) in flight.
template <int MB, int EPI>
__global__ __launch_bounds__(256) void k_gemm_stream(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W,
                                                     int M, int N, int K, int S, Epi e) {
  constexpr int NB = 4, U = 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 64;
  const int s = blockIdx.y;
  const int m0 = blockIdx.z * 16 * MB;
  const int C = K >> 7;
  const int c_beg = (int)((int64_t)s * C / S), c_end = (int)((int64_t)(s + 1) * C / S);
  f32x4 acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bf16_t* wbase = W + (int64_t)(n0 + r) * K + 8 * g;
  const bf16_t* abase[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) abase[mb] = A + (int64_t)min(m0 + 16 * mb + r, M - 1) * K + 8 * g;
  for (int c0 = c_beg + wave; c0 < c_end; c0 += 4 * U) {
    v4u wf[U][NB][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(c0 + 4 * u, c_end - 1);  // a clamped duplicate chunk is loaded, never used
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int st = 0; st < 4; ++st) wf[u][j][st] = *(const v4u*)(wbase + (int64_t)16 * j * K + c * 128 + 32 * st);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 4 * u;
      if (c < c_end) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          v4u af[4];
#pragma unroll
          for (int st = 0; st < 4; ++st) af[st] = *(const v4u*)(abase[mb] + c * 128 + 32 * st);
#pragma unroll
          for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int j = 0; j < NB; ++j) acc[mb][j] = mfma16(af[st], wf[u][j][st], acc[mb][j]);
        }
      }
    }
  }
  __shared__ f32x4 red[3][MB * NB][64];
  if (wave > 0)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < NB; ++j) red[wave - 1][mb * NB + j][lane] = acc[mb][j];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int w = 0; w < 3; ++w) acc[mb][j] += red[w][mb * NB + j][lane];
  }
  Epi ee = e;
  ee.split = s;
  if (wave == 0) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = m0 + 16 * mb + 4 * g + i;
          if (m < M) epi_apply<EPI>(ee, m, n0 + 16 * j + r, acc[mb][j][i]);
        }
  }
}

// M > 64: LDS-staged activations. grid (N/128, S, ceil(M/(16 MB))).
template <int MB, int EPI>
__global__ __launch_bounds__(256) void k_gemm_tile(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W,
                                                   int M, int N, int K, int S, Epi e) {
  constexpr int NB = 2, KC = 64, LDA = KC + 8, ROWS = 16 * MB;
  constexpr int PASSES = ROWS / 32;  // 32 rows x 64 k per 256-thread pass
  static_assert(ROWS % 32 == 0, "tile rows must be a multiple of 32");
  __shared__ bf16_t As[2][ROWS * LDA];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int nw = blockIdx.x * 128 + wave * 32;
  const int s = blockIdx.y;
  const int m0 = blockIdx.z * ROWS;
  const int C = K / KC;
  const int c_beg = (int)((int64_t)s * C / S), c_end = (int)((int64_t)(s + 1) * C / S);
  f32x4 acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const uint4 zero = {0u, 0u, 0u, 0u};
  const int srow = t >> 3, scol = (t & 7) * 8;
  const bf16_t* w0 = W + (int64_t)(nw + r) * K + 8 * g;
  const bf16_t* w1 = w0 + (int64_t)16 * K;

  v4u ast[PASSES];
  v4u wc0[2], wc1[2], wn0[2], wn1[2];
  // prologue: chunk c_beg (every split owns >= 1 chunk)
#pragma unroll
  for (int p = 0; p < PASSES; ++p)
    ast[p] = *(const v4u*)(A + (int64_t)min(m0 + srow + 32 * p, M - 1) * K + c_beg * KC + scol);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    wc0[ks] = *(const v4u*)(w0 + c_beg * KC + 32 * ks);
    wc1[ks] = *(const v4u*)(w1 + c_beg * KC + 32 * ks);
  }
#pragma unroll
  for (int p = 0; p < PASSES; ++p) *(v4u*)(&As[0][(srow + 32 * p) * LDA + scol]) = ast[p];
  for (int c = c_beg; c < c_end; ++c) {
    const int buf = (c - c_beg) & 1;
    // prefetch the next chunk unconditionally (the last iteration re-reads its
    // own chunk) so the staging registers never live across a branch; rows
    // past M are clamped: computed, never stored
    const int cn = min(c + 1, c_end - 1);
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
      ast[p] = *(const v4u*)(A + (int64_t)min(m0 + srow + 32 * p, M - 1) * K + cn * KC + scol);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      wn0[ks] = *(const v4u*)(w0 + cn * KC + 32 * ks);
      wn1[ks] = *(const v4u*)(w1 + cn * KC + 32 * ks);
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const v4u af = *(const v4u*)(&As[buf][(16 * mb + r) * LDA + 32 * ks + 8 * g]);
        acc[mb][0] = mfma16(af, wc0[ks], acc[mb][0]);
        acc[mb][1] = mfma16(af, wc1[ks], acc[mb][1]);
      }
#pragma unroll
    for (int p = 0; p < PASSES; ++p) *(v4u*)(&As[buf ^ 1][(srow + 32 * p) * LDA + scol]) = ast[p];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      wc0[ks] = wn0[ks];
      wc1[ks] = wn1[ks];
    }
  }
  Epi ee = e;
  ee.split = s;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * mb + 4 * g + i;
        if (m < M) epi_apply<EPI>(ee, m, nw + 16 * j + r, acc[mb][j][i]);
      }
}

// ---------------------------------------------------------------------------
// Dispatch
// ---------------------------------------------------------------------------
#define FC_EPI_SWITCH(mode, CALL)                              \
  switch (mode) {                                              \
    case EPI_STORE: { constexpr int E = EPI_STORE; CALL; break; }     \
    case EPI_ADD: { constexpr int E = EPI_ADD; CALL; break; }         \
    case EPI_RELU2: { constexpr int E = EPI_RELU2; CALL; break; }     \
    case EPI_MLPOUT: { constexpr int E = EPI_MLPOUT; CALL; break; }   \
    case EPI_PARTIAL: { constexpr int E = EPI_PARTIAL; CALL; break; } \
    default: { constexpr int E = EPI_SOFTCAP; CALL; break; }          \
  }

template <typename T, int MB>
static void launch_gemv_mb(const void* A, const void* W, int M, int N, int K, const Epi& e, hipStream_t s) {
  const dim3 grid((N + 15) / 16, (M + MB - 1) / MB);
  FC_EPI_SWITCH(e.mode, hipLaunchKernelGGL((k_gemv<T, MB, E>), grid, dim3(256), 0, s, (const T*)A, (const T*)W, M,
                                           N, K, e));
}
template <typename T>
static void launch_gemv(const void* A, const void* W, int M, int N, int K, const Epi& e, hipStream_t s) {
  if (M <= 1) launch_gemv_mb<T, 1>(A, W, M, N, K, e, s);
  else if (M <= 2) launch_gemv_mb<T, 2>(A, W, M, N, K, e, s);
  else if (M <= 4) launch_gemv_mb<T, 4>(A, W, M, N, K, e, s);
  else launch_gemv_mb<T, 8>(A, W, M, N, K, e, s);
}

template <int MB>
static void launch_stream(const void* A, const void* W, int M, int N, int K, int S, const Epi& e, hipStream_t s) {
  const dim3 grid(N / 64, S, (M + 16 * MB - 1) / (16 * MB));
  FC_EPI_SWITCH(e.mode, hipLaunchKernelGGL((k_gemm_stream<MB, E>), grid, dim3(256), 0, s, (const bf16_t*)A,
                                           (const bf16_t*)W, M, N, K, S, e));
}
template <int MB>
static void launch_tile(const void* A, const void* W, int M, int N, int K, int S, const Epi& e, hipStream_t s) {
  const dim3 grid(N / 128, S, (M + 16 * MB - 1) / (16 * MB));
  FC_EPI_SWITCH(e.mode, hipLaunchKernelGGL((k_gemm_tile<MB, E>), grid, dim3(256), 0, s, (const bf16_t*)A,
                                           (const bf16_t*)W, M, N, K, S, e));
}

// split count so that (workgroups x S) reaches ~2 per CU, keeping >= min_chunks
// chunks per split
// split count so that (workgroups x S) reaches ~2 per CU, keeping >= 1 chunk
// per split
static int pick_split(int wgs, int chunks) {
  if (wgs <= 0 || chunks <= 0) return 1;
  int S = (256 + wgs - 1) / wgs;
  return std::max(1, std::min(std::min(S, chunks), FC_MAX_SPLIT));
}

// One plan drives the workspace sizing and the launch.
enum { GK_GEMV = 0, GK_STREAM = 1, GK_TILE = 2 };
struct GemmPlan {
  int kind, mb, mtiles, ntiles, S;
};
static GemmPlan plan_gemm(int M, int N, int K, int dtype, bool can_split) {
  GemmPlan p{};
  p.S = 1;
  if (dtype == FC_F32 || M < 16 || K % 128 != 0 || N % 64 != 0) {
    p.kind = GK_GEMV;
    return p;
  }
  if (M <= 64 || N % 128 != 0) {
    p.kind = GK_STREAM;
    p.mb = std::min(4, (M + 15) / 16);
    p.mtiles = (M + 16 * p.mb - 1) / (16 * p.mb);
    p.ntiles = N / 64;
    if (can_split) p.S = pick_split(p.ntiles * p.mtiles, K / 128);
  } else {
    p.kind = GK_TILE;
    p.ntiles = N / 128;
    // wide N: one M tile streams the weights exactly once; narrower N: 64-row
    // M tiles multiply the workgroups (weight re-reads hit L2 / MALL)
    if (p.ntiles >= 128) p.mb = M <= 128 ? 8 : (M <= 192 ? 12 : (M <= 224 ? 14 : 16));
    else p.mb = 4;
    p.mtiles = (M + 16 * p.mb - 1) / (16 * p.mb);
    if (can_split) p.S = pick_split(p.ntiles * p.mtiles, K / 64);
  }
  return p;
}

int64_t fc_gemm_part_bytes(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  GemmPlan p = plan_gemm(M, N, K, FC_BF16, true);
  return p.S > 1 ? fc_align((int64_t)p.S * M * N * 4) : 0;
}

int fc_launch_gemm(const void* A, const void* W, int M, int N, int K, int dtype, const Epi& e, const GemmWork& gw,
                   hipStream_t s, int* splits) {
  if (splits) *splits = 1;
  if (M <= 0 || N <= 0) return FC_OK;
  FC_CHECK_ARG(K > 0 && K % 8 == 0, "gemm K must be a positive multiple of 8");
  const bool can_split = splits != nullptr && gw.part != nullptr;
  GemmPlan p = plan_gemm(M, N, K, dtype, can_split);
  if (p.S > 1 && (int64_t)p.S * M * N * 4 > gw.part_bytes) p.S = 1;
  Epi ee = e;
  if (p.S > 1) {
    ee.mode = EPI_PARTIAL;
    ee.part = gw.part;
    ee.part_rows = M;
    ee.ldo = N;
    *splits = p.S;
  }
  if (p.kind == GK_GEMV) {
    if (dtype == FC_F32) launch_gemv<float>(A, W, M, N, K, ee, s);
    else launch_gemv<bf16_t>(A, W, M, N, K, ee, s);
  } else if (p.kind == GK_STREAM) {
    if (p.mb == 1) launch_stream<1>(A, W, M, N, K, p.S, ee, s);
    else if (p.mb == 2) launch_stream<2>(A, W, M, N, K, p.S, ee, s);
    else if (p.mb == 3) launch_stream<3>(A, W, M, N, K, p.S, ee, s);
    else launch_stream<4>(A, W, M, N, K, p.S, ee, s);
  } else {
    if (p.mb == 4) launch_tile<4>(A, W, M, N, K, p.S, ee, s);
    else if (p.mb == 8) launch_tile<8>(A, W, M, N, K, p.S, ee, s);
    else if (p.mb == 12) launch_tile<12>(A, W, M, N, K, p.S, ee, s);
    else if (p.mb == 14) launch_tile<14>(A, W, M, N, K, p.S, ee, s);
    else launch_tile<16>(A, W, M, N, K, p.S, ee, s);
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
  return fc_launch_gemm(A, W, M, N, K, dtype, e, GemmWork{}, (hipStream_t)stream, nullptr);
}
