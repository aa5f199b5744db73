// Skinny GEMMs with fused epilogues: out = epi(A[M][K] . W[N][K]^T).
//
// Replaces the nnx.Linear matmuls of the per-token forward
// (flaxchat/engine.py:106-108, 158, 161, 172; flaxchat/gpt.py:93-99, 154-163)
// and fuses what the reference does right after them: the residual add
// (engine.py:160-161), ReLU^2 (gpt.py:161), resid/x0 lambda mix of the next
// layer (engine.py:94), the backout capture and subtraction
// (engine.py:164-166) and the 15*tanh(z/15) softcap (engine.py:173-174).
//
// Kernels:
//   k_gemv     VALU dot products (fp32 weights: the parity mode).
//   k_gemm_ks  bf16 MFMA 16x16x32, workgroup tile of 16-32 rows x 16-64
//              columns, the four waves split K, register pipeline; draft
//              steps and the split-K residual GEMMs.
//   k_gemm_la  bf16 MFMA, 32-128 rows x 128 columns, the four waves split
//              the columns and share the activation tile through LDS;
//              verify row counts, the QKV GEMM with its fused attention
//              prologue (also at one-row decode sizes) and the draft lm_head.
//   k_gemm_dma bf16 MFMA, 64 x 64 tiles fed by direct global-to-LDS loads
//              into a 4-stage ring; verify c_fc.
//   k_gemm_ring bf16 MFMA, 64 x 96 tiles, a 5-stage direct-load LDS ring;
//              the verify MLP c_proj (K split 4).
//   k_gemm_big bf16 MFMA, 256 x 256 tiles, 4-stage LDS ring of direct
//              loads; prefill chunks (M >= 1024) and the lm_head from 200
//              rows (the verify head).
// The row count may be a device value (packed token chunks whose size is
// only known on the GPU): the grid covers the capacity and tiles past the
// actual count exit at once.
// When N alone gives too few workgroups to occupy 256 CUs, a GEMM whose
// output is the fp32 residual stream may split K across workgroups: each
// split writes its partial product with plain stores and the RMSNorm kernel
// that consumes x next sums the splits in fixed order and applies the
// epilogue (a kernel boundary is the only synchronisation; on MI355X the
// eight XCD L2 caches are not coherent, so an in-kernel device-scope fence
// would write back a whole L2 per workgroup).
#include "fc_common.h"
#include "fc_internal.h"

// 15 tanh(v / 15) in the bf16 kernels' epilogues. tanh(x) = sign(x) (1 - 2 /
// (e^{2|x|} + 1)) with e^{2|x|} from the hardware base-2 exponential and the
// reciprocal from v_rcp_f32 (about 1 ulp each); below |x| = 1/16, where that
// form cancels, the series x - x^3/3 + 2x^5/15 (truncation < 3e-10). The
// capped value is within ~5e-6 of 15 tanhf(v / 15), far below the bf16
// GEMM's own rounding, at about a third of the instructions of the
// IEEE divide and tanhf. The fp32 kernels keep the exact form.
__device__ __forceinline__ float softcap15_fast(float v) {
  const float x = v * (1.f / 15.f);
  const float a = fabsf(x);
  const float x2 = x * x;
  const float ts = x * fmaf(x2, fmaf(x2, 2.f / 15.f, -1.f / 3.f), 1.f);
  const float ex = __builtin_amdgcn_exp2f(a * 2.8853900817779268f);  // e^{2a}
  const float tl = copysignf(1.f - 2.f * __builtin_amdgcn_rcpf(ex + 1.f), x);
  return 15.f * (a < 0.0625f ? ts : tl);
}

// FAST: the bf16 kernels' softcap (softcap15_fast); the fp32 kernel uses tanhf.
template <int EPI, bool FAST = false>
__device__ __forceinline__ void epi_apply(const Epi e, int m, int n, float acc) {
  if constexpr (EPI == EPI_STORE) {
    ((float*)e.out)[(int64_t)m * e.ldo + n] = acc;
  } else if constexpr (EPI == EPI_ADD) {
    float* o = (float*)e.out + (int64_t)m * e.ldo + n;
    *o = *o + acc;
  } else if constexpr (EPI == EPI_RELU2) {  // the next GEMM's operand: fragment order in bf16
    float r = fmaxf(acc, 0.f);
    r = r * r;
    if (e.out_dtype == FC_BF16) ((bf16_t*)e.out)[frag_idx(m, n, (int)e.ldo)] = f2bf(r);
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
      ((float*)e.out)[(int64_t)b * e.row_stride + (int64_t)rr * e.V + n] =
          FAST ? softcap15_fast(acc) : 15.f * tanhf(acc / 15.f);
    }
  }
}

// Folded RMSNorm, consumer side: the 256 / MT threads of each output row
// (consecutive lanes) each load up to FC_RMS_REG of the row's per-tile sums
// of squares at kernel start (clamped, unconditional: one batch of loads in
// flight together) and keep them in registers through the K loop, whose
// loads they precede; the epilogue adds them up over those lanes (a fixed
// shuffle tree: deterministic).
#define FC_RMS_REG 16
struct RmsPre {
  float v[FC_RMS_REG];
};
template <int MT>
__device__ __forceinline__ void rms_load(RmsPre& r, const Epi& e, int m0, int M) {
  constexpr int TPR = 256 / MT;
  const int m = min(m0 + (int)threadIdx.x / TPR, M - 1), sub = (int)threadIdx.x % TPR;
#pragma unroll
  for (int j = 0; j < FC_RMS_REG; ++j) r.v[j] = e.rms_in[(int64_t)min(sub + j * TPR, e.rms_n - 1) * e.ssq_ld + m];
}
template <int MT>
__device__ __forceinline__ float rms_finish(const RmsPre& r, const Epi& e, int K) {
  constexpr int TPR = 256 / MT;
  const int sub = (int)threadIdx.x % TPR;
  float p = 0.f;
#pragma unroll
  for (int j = 0; j < FC_RMS_REG; ++j) p += sub + j * TPR < e.rms_n ? r.v[j] : 0.f;
#pragma unroll
  for (int o = TPR / 2; o > 0; o >>= 1) p += __shfl_xor(p, o, WAVE);
  return 1.f / sqrtf(p / (float)K + 1e-6f);
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
__global__ __launch_bounds__(256) void k_gemv(const T* __restrict__ A, const T* __restrict__ W, int Mcap,
                                              const int* __restrict__ Mdev, int N, int K, Epi e) {
  constexpr int VEC = 16 / sizeof(T);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wave) * 4;
  const int m0 = blockIdx.y * MB;
  const int M = Mdev ? min(*Mdev, Mcap) : Mcap;
  if (m0 >= M) return;
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
// weight fragment loads: plain (they are re-read across M tiles through L2)
#define W_LD(p) (*(p))
// lm_head weights (the softcap epilogue) always stream non-temporally: the
// matrix (201 MB at cfg4) is about the size of the 256 MB Infinity Cache,
// and both the verify and the draft lm_head reading it non-temporally made
// the speculative round 2.2% faster (5.01 -> 4.91 ms) than either one alone
// or neither (the other reads of the round keep their cache lines). The
// other GEMMs re-read weight tiles across M tiles through L2 and lose more
// than they gain from it (5.0 -> 5.3 ms).
#define LM_LD(p) __builtin_nontemporal_load(p)
// The same for the lm_head on the K-split kernel (one-row decode: cfg2's
// 100 MB head read five times a round; 0.917-0.918 vs 0.924 ms per round)
// and on the 256 x 256 kernel's direct loads (the cfg4 verify head:
// 4.835-4.837 vs 4.840-4.845 ms per round), alternating builds.
#ifndef FC_KS_LM_NT
#define FC_KS_LM_NT 1
#endif
#ifndef FC_BIG_LM_NT
#define FC_BIG_LM_NT 1
#endif
__device__ __forceinline__ f32x4 mfma16(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                  0, 0);
}
__device__ __forceinline__ f32x4 mfma16(v4u a, v4u b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                  0, 0);
}

// Epilogue on finished sums laid out row-major: thread t owns OPT = MT NT /
// 256 consecutive columns col0 .. of tile row `row` = t / (NT / OPT) (the
// threads of a row are consecutive lanes). Used by the kernels that stage
// their tile in LDS first (k_gemm_ks, k_gemm_ring): the folded-norm
// epilogues need whole row segments per thread.
template <int EPI, int MT, int NT>
__device__ __forceinline__ void row_epilogue(const Epi& e, float (&v)[MT * NT / 256], int row, int col0, int m0,
                                             int n0, int nt, int s, int M, int K, const RmsPre& rpre) {
  constexpr int OPT = MT * NT / 256, TPR = NT / OPT;
  const int m = m0 + row;
  const bool live = m < M;
  if constexpr (EPI == EPI_RELU2) {
    if (e.rms_in != nullptr) {  // thread t's epilogue row is its prefetch row (t / TPR)
      static_assert(TPR == 256 / MT, "row mapping");
      const float sc = rms_finish<MT>(rpre, e, K);
#pragma unroll
      for (int c = 0; c < OPT; ++c) v[c] *= sc;
    }
  }
  if constexpr (EPI == EPI_ADD) {
    if (e.xa != nullptr) {
      // residual add, bf16 copy of the new x (OPT consecutive columns: whole
      // bf16 pairs in fragment order) and the row's sum of squares over this
      // tile (the TPR threads of a row are consecutive lanes)
      static_assert(OPT % 2 == 0 && 64 % TPR == 0, "folded-norm epilogue tiling");
      float ss = 0.f;
      if (live) {
        float* o = (float*)e.out + (int64_t)m * e.ldo + n0 + col0;
#pragma unroll
        for (int c = 0; c < OPT; c += 2) {
          const float a0 = o[c] + v[c], a1 = o[c + 1] + v[c + 1];
          o[c] = a0;
          o[c + 1] = a1;
          ss += a0 * a0 + a1 * a1;
          *(uint32_t*)(e.xa + frag_idx(m, n0 + col0 + c, (int)e.ldo)) =
              (uint32_t)f2bf(a0) | ((uint32_t)f2bf(a1) << 16);
        }
      }
#pragma unroll
      for (int o = TPR / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, WAVE);
      if (live && col0 == 0) e.ssq[(int64_t)nt * e.ssq_ld + m] = ss;
      return;
    }
  }
  if (!live) return;
  Epi ee = e;
  ee.split = s;
#pragma unroll
  for (int c = 0; c < OPT; ++c) epi_apply<EPI, true>(ee, m, n0 + col0 + c, v[c]);
}

// bf16 MFMA GEMM, K split over the four waves of a workgroup.
//
// A workgroup owns an MT x NT output tile (MT = 16 MB rows, NT = 16 NB
// columns) over its split's K range; its four waves take interleaved
// 64-wide k chunks, so every weight and activation byte reaches the CU once
// and no LDS traffic or barrier sits in the main loop. Each wave keeps NS
// chunks of A and W fragments in flight in registers (the loads of chunk
// i + NS are issued right after chunk i is consumed). The four partial
// tiles are summed in LDS at the end and the epilogue runs on a coalesced
// row-major layout.
//
// Grid: 1-D over (N tile, K split, M tile), the N tile count padded to a
// multiple of 8. Workgroups are dealt to the eight XCDs round robin and both
// tile orders keep N tile n on XCD n % 8, so the M tiles that share its
// weight slab read it from HBM once and hit in that XCD's L2:
//   mfast = 1: within an XCD the M tiles of one N tile run back to back
//              (wide N, e.g. lm_head: the slab is reused while still in L2);
//   mfast = 0: M tile slowest; with a device row count (`Mdev`, at most
//              Mcap) the tiles past it come last in dispatch order and exit
//              at once.
template <int MB, int NB, int NS, int EPI, bool PK = false>
__global__ __launch_bounds__(256) void k_gemm_ks(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W,
                                                 int Mcap, const int* __restrict__ Mdev, int N, int K, int ntiles,
                                                 int S, int mtiles, int mfast, Epi e) {
  constexpr int MT = 16 * MB, NT = 16 * NB;
  const int id = blockIdx.x;
  const int ntiles8 = (ntiles + 7) & ~7;
  int nt, s, mt;
  if (mfast) {  // per XCD: the M tiles of one N tile back to back
    const int xcd = id & 7, loc = id >> 3, per = S * mtiles;
    const int nl = loc / per, rem = loc - nl * per;
    s = rem / mtiles;
    mt = rem - s * mtiles;
    nt = nl * 8 + xcd;
  } else {      // M tile slowest
    nt = id % ntiles8;
    const int rest = id / ntiles8;
    s = rest % S;
    mt = rest / S;
  }
  if (nt >= ntiles) return;
  const int M = Mdev ? min(*Mdev, Mcap) : Mcap;
  const int m0 = mt * MT;
  if (m0 >= M) return;
  const int n0 = nt * NT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int C = K >> 6;
  const int c_beg = (int)((int64_t)s * C / S), c_end = (int)((int64_t)(s + 1) * C / S);
  const int nch = c_end - c_beg > wave ? (c_end - c_beg - wave + 3) >> 2 : 0;
  RmsPre rpre;  // folded RMSNorm: this thread's share of its output row's sums of squares
  if constexpr (EPI == EPI_RELU2) {
    if (e.rms_in != nullptr) rms_load<MT>(rpre, e, m0, M);
  }

  f32x4 acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // operand addresses at k = 0. Row-major: lane l reads row (l % 16), 16 B
  // at k = 8 (l / 16). Fragment order (PK): 16-row x 32-k blocks of 1 KB in
  // [row block][k step] order, lane l's 16 B at offset 16 l of its block,
  // so each load instruction reads 1 KB contiguous. Either way the chunk
  // offset of k step t is `kstep_elems * t`.
  const bf16_t* wrow[NB];
  const bf16_t* arow[MB];
  int64_t kstep_elems;
  if constexpr (PK) {
    const int64_t KS32 = K >> 5;
#pragma unroll
    for (int j = 0; j < NB; ++j) wrow[j] = W + (int64_t)(n0 / 16 + j) * KS32 * 512 + lane * 8;
    const int last_blk = (M - 1) >> 4;
#pragma unroll
    for (int i = 0; i < MB; ++i) arow[i] = A + (int64_t)min(m0 / 16 + i, last_blk) * KS32 * 512 + lane * 8;
    kstep_elems = 512;
  } else {
#pragma unroll
    for (int j = 0; j < NB; ++j) wrow[j] = W + (int64_t)(n0 + 16 * j + r) * K + 8 * g;
#pragma unroll
    for (int i = 0; i < MB; ++i) arow[i] = A + (int64_t)min(m0 + 16 * i + r, M - 1) * K + 8 * g;
    kstep_elems = 32;
  }

  if (nch > 0) {
    static_assert(NS >= 2 && NS <= 4, "register ring of 2-4 chunks");
    v4u wb[NS][NB][2], ab[NS][MB][2];
    // chunk index of the wave's i-th chunk, clamped so the tail loads are
    // harmless re-reads and the loop body has no branch
#define KS_LOAD(slot, i)                                                            \
  {                                                                                 \
    const int c_ = c_beg + wave + 4 * min((i), nch - 1);                            \
    _Pragma("unroll") for (int j = 0; j < NB; ++j)                                  \
      _Pragma("unroll") for (int ks = 0; ks < 2; ++ks)                              \
        wb[slot][j][ks] = EPI == EPI_SOFTCAP && FC_KS_LM_NT ? LM_LD((const v4u*)(wrow[j] + (2 * c_ + ks) * kstep_elems)) \
                                                             : W_LD((const v4u*)(wrow[j] + (2 * c_ + ks) * kstep_elems)); \
    _Pragma("unroll") for (int mb = 0; mb < MB; ++mb)                               \
      _Pragma("unroll") for (int ks = 0; ks < 2; ++ks)                              \
        ab[slot][mb][ks] = *(const v4u*)(arow[mb] + (2 * c_ + ks) * kstep_elems);   \
  }
#define KS_MMA(slot)                                                                \
  {                                                                                 \
    _Pragma("unroll") for (int ks = 0; ks < 2; ++ks)                                \
      _Pragma("unroll") for (int mb = 0; mb < MB; ++mb)                             \
        _Pragma("unroll") for (int j = 0; j < NB; ++j)                              \
          acc[mb][j] = mfma16(ab[slot][mb][ks], wb[slot][j][ks], acc[mb][j]);       \
  }
#pragma unroll
    for (int p = 0; p < NS; ++p) KS_LOAD(p, p);
    int i = 0;
    // the scheduling barriers keep each chunk's loads together and after the
    // MFMAs that free its registers, so the other slots' loads stay in flight
    // while a slot computes (the waits become vmcnt(NS - 1 slots))
    for (; i + NS - 1 < nch; i += NS) {
#pragma unroll
      for (int p = 0; p < NS; ++p) {
        KS_MMA(p);
        __builtin_amdgcn_sched_barrier(0);
        KS_LOAD(p, i + NS + p);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // the last nch - i < NS chunks sit in slots 0 .. nch - i - 1
#pragma unroll
    for (int p = 0; p < NS - 1; ++p)
      if (i + p < nch) KS_MMA(p);
#undef KS_LOAD
#undef KS_MMA
  }

  // sum the four waves' tiles; thread t then owns OPT consecutive columns
  // of one row
  constexpr int LDR = NT + 4, OPT = MT * NT / 256, TPR = NT / OPT;
  static_assert(OPT >= 1 && NT % OPT == 0, "epilogue tiling");
  __shared__ float red[4][MT][LDR];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave][16 * mb + 4 * g + i][16 * j + r] = acc[mb][j][i];
  __syncthreads();
  const int t = threadIdx.x;
  const int row = t / TPR, col0 = (t - row * TPR) * OPT;
  float v[OPT];
#pragma unroll
  for (int c = 0; c < OPT; ++c)
    v[c] = red[0][row][col0 + c] + red[1][row][col0 + c] + red[2][row][col0 + c] + red[3][row][col0 + c];
  row_epilogue<EPI, MT, NT>(e, v, row, col0, m0, n0, nt, s, M, K, rpre);
}

// Attention prologue of one token and one head slot from its fp32 GEMM
// output row x (128 values; flaxchat/engine.py:96-126, flaxchat/gpt.py:65-71):
// q / k heads get RoPE (pairs d, d + 64) and 1.2 * RMSNorm, v heads the
// value-embedding gate; q goes to q[m][head], k / v to the cache at the
// token's position. Eight consecutive lanes share a token (`part` = which
// 8 rotary pairs); all 8 take part in the norm's shuffles.
//
// The inputs that do not depend on the GEMM result are loaded first, in two
// steps that callers issue ahead of the accumulator staging so the loads of
// several tokens are in flight together: qkv_pre_row (the token's cache row,
// position and id) and qkv_pre_tab (the rotary table entries of the q / k
// heads; the value-embedding slice and the gate inputs of the v heads).
struct QkvPre {
  int b, pos, tok;
  float c[8], s[8];  // q / k heads: cos / sin of the lane's 8 rotary pairs
  uint4 h0, ve0, ve1;  // v heads: A row k 0..7, ve dims 8 part .. +7 and 64 + 8 part .. +7
  uint2 h1;            // v heads: A row k 8..11
};

__device__ __forceinline__ void qkv_pre_row(const QkvEpi& Q, int m, int M, int hh, QkvPre& p) {
  p.b = 0;
  p.pos = 0;
  p.tok = 0;
  if (m < M) {
    p.b = Q.tok_row[m];
    p.pos = Q.tok_pos[m];
    if (hh >= Q.H + Q.G && Q.ve != nullptr) p.tok = Q.tokens[m];
  }
}

__device__ __forceinline__ void qkv_pre_tab(const QkvEpi& Q, int m, int M, int hh, int part, QkvPre& p) {
  if (hh < Q.H + Q.G) {
    const int pc = min(max(p.pos, 0), Q.rope_len - 1);
    const float4* cp = (const float4*)(Q.rcos + (int64_t)pc * 64 + 8 * part);
    const float4* sp = (const float4*)(Q.rsin + (int64_t)pc * 64 + 8 * part);
    const float4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
    p.c[0] = c0.x; p.c[1] = c0.y; p.c[2] = c0.z; p.c[3] = c0.w;
    p.c[4] = c1.x; p.c[5] = c1.y; p.c[6] = c1.z; p.c[7] = c1.w;
    p.s[0] = s0.x; p.s[1] = s0.y; p.s[2] = s0.z; p.s[3] = s0.w;
    p.s[4] = s1.x; p.s[5] = s1.y; p.s[6] = s1.z; p.s[7] = s1.w;
  } else if (Q.ve != nullptr && m < M) {
    // A row m, k 0..7 then 8..11: 16 contiguous bytes each in fragment order
    const uint16_t* hr = Q.h + frag_idx(m, 0, Q.D);
    p.h0 = *(const uint4*)hr;
    p.h1 = *(const uint2*)(hr + 128);
    const uint16_t* vr = Q.ve + ((int64_t)p.tok * Q.G + (hh - Q.H - Q.G)) * 128;
    p.ve0 = *(const uint4*)(vr + 8 * part);
    p.ve1 = *(const uint4*)(vr + 64 + 8 * part);
  }
}

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ void qkv_finish(const QkvEpi& Q, const float* x, int m, int M, int hh, int part,
                                           const QkvPre& p) {
  const bool live = m < M;
  float x1[8], x2[8];
  {
    const float4* xa = (const float4*)(x + 8 * part);
    const float4* xb = (const float4*)(x + 64 + 8 * part);
    const float4 a0 = xa[0], a1 = xa[1], b0 = xb[0], b1 = xb[1];
    x1[0] = a0.x; x1[1] = a0.y; x1[2] = a0.z; x1[3] = a0.w; x1[4] = a1.x; x1[5] = a1.y; x1[6] = a1.z; x1[7] = a1.w;
    x2[0] = b0.x; x2[1] = b0.y; x2[2] = b0.z; x2[3] = b0.w; x2[4] = b1.x; x2[5] = b1.y; x2[6] = b1.z; x2[7] = b1.w;
  }
  const int b = p.b, pos = p.pos;
  // a token whose row lies outside [0, B) (an empty or rejected chunk row)
  // writes nothing, q included, like the unfused prologue
  const bool in_row = live && (unsigned)b < (unsigned)Q.B;
  const bool in_cache = in_row && pos >= 0 && pos < Q.cap;
  if (hh < Q.H + Q.G) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float c = p.c[e], s = p.s[e];
      const float y1 = x1[e] * c + x2[e] * s;
      const float y2 = x1[e] * (-s) + x2[e] * c;
      x1[e] = y1;
      x2[e] = y2;
      ss += y1 * y1 + y2 * y2;
    }
    ss += __shfl_xor(ss, 1, WAVE);
    ss += __shfl_xor(ss, 2, WAVE);
    ss += __shfl_xor(ss, 4, WAVE);
    const float inv = 1.f / sqrtf(ss / 128.f + 1e-6f);
    uint4 p1, p2;
    uint32_t* w1 = (uint32_t*)&p1;
    uint32_t* w2 = (uint32_t*)&p2;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      w1[e] = (uint32_t)f2bf(x1[2 * e] * inv * 1.2f) | ((uint32_t)f2bf(x1[2 * e + 1] * inv * 1.2f) << 16);
      w2[e] = (uint32_t)f2bf(x2[2 * e] * inv * 1.2f) | ((uint32_t)f2bf(x2[2 * e + 1] * inv * 1.2f) << 16);
    }
    if (hh < Q.H) {
      if (in_row) {
        bf16_t* qo = Q.q + ((int64_t)m * Q.H + hh) * 128;
        *(uint4*)(qo + 8 * part) = p1;
        *(uint4*)(qo + 64 + 8 * part) = p2;
      }
    } else if (in_cache) {
      bf16_t* kg = Q.kc + ((int64_t)b * Q.G + (hh - Q.H)) * Q.cap * 128;
      *(uint4*)(kg + kblk_idx(pos, 8 * part)) = p1;       // 8 consecutive dims stay contiguous
      *(uint4*)(kg + kblk_idx(pos, 64 + 8 * part)) = p2;
    }
  } else {
    const int gv = hh - Q.H - Q.G;
    if (Q.ve != nullptr && live) {
      const uint32_t hw[6] = {p.h0.x, p.h0.y, p.h0.z, p.h0.w, p.h1.x, p.h1.y};
      const float* wg = Q.ve_gate + gv * 12;
      float z = 0.f;
#pragma unroll
      for (int i = 0; i < 6; ++i) {
        z += bf_lo(hw[i]) * wg[2 * i];
        z += bf_hi(hw[i]) * wg[2 * i + 1];
      }
      const float gate = 3.f * (1.f / (1.f + expf(-z)));
      const uint32_t va[4] = {p.ve0.x, p.ve0.y, p.ve0.z, p.ve0.w}, vb[4] = {p.ve1.x, p.ve1.y, p.ve1.z, p.ve1.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x1[2 * e] = x1[2 * e] + gate * bf_lo(va[e]);
        x1[2 * e + 1] = x1[2 * e + 1] + gate * bf_hi(va[e]);
        x2[2 * e] = x2[2 * e] + gate * bf_lo(vb[e]);
        x2[2 * e + 1] = x2[2 * e + 1] + gate * bf_hi(vb[e]);
      }
    }
    if (in_cache) {
      bf16_t* vb = Q.vc + (((int64_t)b * Q.G + gv) * (Q.cap / 32) + pos / 32) * 128 * 32 + (pos & 31);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        vb[(8 * part + e) * 32] = f2bf(x1[e]);
        vb[(64 + 8 * part + e) * 32] = f2bf(x2[e]);
      }
    }
  }
}

// The draw's Gumbel noise for this thread's epilogue columns (row m0 + t / 8,
// NT / 8 columns from n0 + (t % 8) NT / 8), which depends only on the Philox
// counter: where the tile has a single 32-row pass (MB = 2) k_gemm_la computes
// it before its K loop, while the first chunks load, instead of in the tail.
template <int MB, int NBW>
struct VpNoise {
  float g[MB == 2 ? 8 * NBW : 1];
  bool ok;
};
template <int MB, int NBW>
__device__ __forceinline__ bool vp_noise_wanted(const Epi& e) {
  return MB == 2 && e.vp != nullptr && e.vp_draw && e.vp_T > 0.f;
}
template <int MB, int NBW>
__device__ __forceinline__ void vp_noise(const Epi& e, int m0, int n0, int rnd, VpNoise<MB, NBW>& nz) {
  nz.ok = false;
  if constexpr (MB == 2) {
    if (!vp_noise_wanted<MB, NBW>(e)) return;
    constexpr int PER = 8 * NBW;
    const int m = m0 + (threadIdx.x >> 3), c0 = n0 + (threadIdx.x & 7) * PER;
#pragma unroll
    for (int w0 = 0; w0 < PER; w0 += 4) {
      const u32x4 rr = philox4x32_10(u32x4{(uint32_t)((c0 + w0) >> 2), (uint32_t)m, (uint32_t)rnd,
                                           (uint32_t)e.vp_slot},
                                     (uint32_t)e.vp_seed, (uint32_t)(e.vp_seed >> 32));
#pragma unroll
      for (int w = 0; w < 4; ++w) nz.g[w0 + w] = gumbel_of(pick(rr, w));
    }
    nz.ok = true;
  }
}

// Vocab-pass partials of the logits tile (EPI_SOFTCAP with e.vp): the same
// terms as the separate pass (k_vpart) over the tile's columns instead of a
// 1024-entry chunk, so the draft step needs no second pass over its logits.
// Per 32 rows the capped values are staged in LDS; then 8 consecutive lanes
// own a row, NT / 8 columns each (whole Philox groups of 4), and reduce with
// shuffles; lane 0 of the 8 writes the row's VPart.
// The capped logits are stored here too, from the same values the partials
// are computed from (acc is overwritten with them).
template <int MB, int NBW>
__device__ __forceinline__ void vocab_tile_parts(const Epi& e, f32x4 (&acc)[MB][NBW], int m0, int n0, int nt,
                                                 int M, const VpNoise<MB, NBW>* nz) {
  constexpr int NT = 64 * NBW, PER = NT / 8, LD = NT + 4;
  static_assert(MB % 2 == 0, "32-row passes");
  __shared__ __align__(16) float T[32 * LD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int row = threadIdx.x >> 3, q = threadIdx.x & 7;
  const int c0 = n0 + q * PER;  // this thread's first column
  const float Tt = e.vp_T;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < NBW; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float z = softcap15_fast(acc[mb][j][i]);
        acc[mb][j][i] = z;
        const int m = m0 + 16 * mb + 4 * g + i, n = n0 + 16 * (wave * NBW + j) + r;
        if (m < M && n < e.V) {
          const int b = m / e.n_out, rr = m - b * e.n_out;
          ((float*)e.out)[(int64_t)b * e.row_stride + (int64_t)rr * e.V + n] = z;
        }
      }
#pragma unroll
  for (int p = 0; p < MB / 2; ++p) {
    if (p > 0) __syncthreads();  // the previous pass's readers are done with T
#pragma unroll
    for (int mh = 0; mh < 2; ++mh)
#pragma unroll
      for (int j = 0; j < NBW; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) T[(16 * mh + 4 * g + i) * LD + 16 * (wave * NBW + j) + r] = acc[2 * p + mh][j][i];
    __syncthreads();
    const int m = m0 + 32 * p + row;
    float v[PER];
#pragma unroll
    for (int w = 0; w < PER; w += 4) {
      const float4 t4 = *reinterpret_cast<const float4*>(&T[row * LD + q * PER + w]);
      v[w] = t4.x;
      v[w + 1] = t4.y;
      v[w + 2] = t4.z;
      v[w + 3] = t4.w;
    }
    float bz = -INFINITY;
    int bzi = 0x7fffffff;
#pragma unroll
    for (int w = 0; w < PER; ++w)
      if (c0 + w < e.V) argmax_merge(bz, bzi, v[w], c0 + w);
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) argmax_merge(bz, bzi, __shfl_xor(bz, o, WAVE), __shfl_xor(bzi, o, WAVE));
    VPart pt;
    pt.zmax = bz;
    pt.zarg = bzi;
    pt.m = 0.f;
    pt.s = 1.f;
    pt.a = -INFINITY;
    pt.ai = 0x7fffffff;
    pt.g = -INFINITY;
    pt.gi = 0x7fffffff;
    if (Tt > 0.f) {
      const float mx = bz / Tt;
#pragma unroll
      for (int w = 0; w < PER; ++w) v[w] = v[w] / Tt;
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < PER; ++w)
        if (c0 + w < e.V) sum += expf(v[w] - mx);
#pragma unroll
      for (int o = 1; o < 8; o <<= 1) sum += __shfl_xor(sum, o, WAVE);
      pt.m = mx;
      pt.s = sum;
      if (e.vp_draw) {
        const int rnd = m < M ? e.vp_round[m] : 0;
        float ba = -INFINITY, bg = -INFINITY;
        int bai = 0x7fffffff, bgi = 0x7fffffff;
        bool pre = false;
        if constexpr (MB == 2) {
          if (nz != nullptr && nz->ok) {  // the noise computed before the K loop
            pre = true;
#pragma unroll
            for (int w = 0; w < PER; ++w) {
              const int i = c0 + w;
              if (i >= e.V) break;
              argmax_merge(ba, bai, (v[w] - mx) + nz->g[w], i);
              argmax_merge(bg, bgi, nz->g[w], i);
            }
          }
        }
        if (!pre) {
#pragma unroll
          for (int w0 = 0; w0 < PER; w0 += 4) {
            if (c0 + w0 >= e.V) break;
            const u32x4 rr = philox4x32_10(u32x4{(uint32_t)((c0 + w0) >> 2), (uint32_t)m, (uint32_t)rnd,
                                                 (uint32_t)e.vp_slot},
                                           (uint32_t)e.vp_seed, (uint32_t)(e.vp_seed >> 32));
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              const int i = c0 + w0 + w;
              if (i >= e.V) break;
              const float G = gumbel_of(pick(rr, w));
              argmax_merge(ba, bai, (v[w0 + w] - mx) + G, i);
              argmax_merge(bg, bgi, G, i);
            }
          }
        }
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) {
          argmax_merge(ba, bai, __shfl_xor(ba, o, WAVE), __shfl_xor(bai, o, WAVE));
          argmax_merge(bg, bgi, __shfl_xor(bg, o, WAVE), __shfl_xor(bgi, o, WAVE));
        }
        pt.a = ba;
        pt.ai = bai;
        pt.g = bg;
        pt.gi = bgi;
      }
    }
    if (q == 0 && m < M) {
      float4* dst = reinterpret_cast<float4*>(e.vp + (int64_t)m * e.vp_ld + nt);
      dst[0] = make_float4(pt.zmax, __int_as_float(pt.zarg), pt.m, pt.s);
      dst[1] = make_float4(pt.a, __int_as_float(pt.ai), pt.g, __int_as_float(pt.gi));
    }
  }
}

// Epilogue of the column-split kernels (k_gemm_la, k_gemm_dma): acc[mb][j]
// holds rows 16 mb + 4 g + i, column 16 (wave NBW + j) + r of the tile. VP:
// the kernel can write the vocab-pass partials (k_gemm_la).
template <int MB, int NBW, int EPI, bool VP = false>
__device__ __forceinline__ void tile_epilogue(const Epi& e, const f32x4 (&acc)[MB][NBW], const RmsPre& rpre,
                                              QkvPre (&qpre)[(MB + 1) / 2], int m0, int n0, int nt, int s, int M,
                                              int K, const VpNoise<MB, NBW>* nz = nullptr) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  if constexpr (EPI == EPI_QKV) {
    // the tile is one head (column tile nt = head slot) for 32 or 64 tokens:
    // per 32 tokens, stage them in LDS, then 8 threads per token finish them
    // (16 dims each: d and d + 64 of 8 rotary pairs)
    static_assert((MB == 2 || MB == 4) && NBW == 2, "EPI_QKV needs 32 x 128 or 64 x 128 tiles");
    __shared__ float T[32][128 + 4];
#pragma unroll
    for (int p = 0; p < MB / 2; ++p) {
      const int mt = m0 + 32 * p + (threadIdx.x >> 3);
      qkv_pre_tab(e.qkv, mt, M, nt, threadIdx.x & 7, qpre[p]);  // in flight while staging
      if (p > 0) __syncthreads();  // the previous pass's readers are done with T
#pragma unroll
      for (int mh = 0; mh < 2; ++mh)
#pragma unroll
        for (int j = 0; j < NBW; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) T[16 * mh + 4 * g + i][16 * (wave * NBW + j) + r] = acc[2 * p + mh][j][i];
      __syncthreads();
      qkv_finish(e.qkv, T[threadIdx.x >> 3], mt, M, nt, threadIdx.x & 7, qpre[p]);
    }
  } else {
    // folded RMSNorm (RELU2 reading the bf16 copy of x): acc row
    // 16 mb + 4 g + i takes the factor lane 4 g + i computed for its row
    float rsc[MB][4];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) rsc[mb][i] = 1.f;
    if constexpr (EPI == EPI_RELU2) {
      if (e.rms_in != nullptr) {
        constexpr int MT = 16 * MB;
        __shared__ float rowinv[MT];
        const float inv = rms_finish<MT>(rpre, e, K);
        if (threadIdx.x % (256 / MT) == 0) rowinv[threadIdx.x / (256 / MT)] = inv;
        __syncthreads();
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int i = 0; i < 4; ++i) rsc[mb][i] = rowinv[16 * mb + 4 * g + i];
      }
    }
    if constexpr (VP && EPI == EPI_SOFTCAP && MB % 2 == 0) {
      if (e.vp != nullptr) {
        f32x4 z[MB][NBW];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int j = 0; j < NBW; ++j) z[mb][j] = acc[mb][j];
        vocab_tile_parts<MB, NBW>(e, z, m0, n0, nt, M, nz);
        return;
      }
    }
    Epi ee = e;
    ee.split = s;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < NBW; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = m0 + 16 * mb + 4 * g + i;
          if (m < M) epi_apply<EPI, true>(ee, m, n0 + 16 * (wave * NBW + j) + r, acc[mb][j][i] * rsc[mb][i]);
        }
  }
}

// bf16 MFMA GEMM for larger row counts, A shared through LDS.
//
// A workgroup owns an MT x NT tile (MT = 16 MB rows, NT = 64 NBW columns);
// its four waves split the columns (each 16 NBW of them, all MT rows), so
// each wave streams only its own weight fragments, straight into registers,
// while the activation tile of a 64-wide k chunk (2 MB blocks of 1 KB in
// fragment order) is fetched once per workgroup and shared in LDS. Per
// output this moves (MT + NT) / (MT NT) of the operand bytes through L2,
// half of what the K-split kernel's 32 x 64 tile moves at MT = 64, NT = 128.
// Both operands are loaded NS chunks ahead in a register ring; the A chunk
// is written to the LDS double buffer one chunk before it is used.
// Grid and tile order as in k_gemm_ks.
template <int MB, int NBW, int NS, int EPI>
__global__ __launch_bounds__(256) void k_gemm_la(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W,
                                                 int Mcap, const int* __restrict__ Mdev, int N, int K, int ntiles,
                                                 int S, int mtiles, int mfast, Epi e) {
  static_assert(MB == 2 || MB == 4 || MB == 8 || MB == 16, "MB in {2, 4, 8, 16}");
  constexpr int MT = 16 * MB, NT = 64 * NBW, AB = 2 * MB / 4;  // A blocks per wave per chunk
  __shared__ uint4 As[2][2 * MB][64];
  const int id = blockIdx.x;
  const int ntiles8 = (ntiles + 7) & ~7;
  int nt, s, mt;
  if (mfast) {
    const int xcd = id & 7, loc = id >> 3, per = S * mtiles;
    const int nl = loc / per, rem = loc - nl * per;
    s = rem / mtiles;
    mt = rem - s * mtiles;
    nt = nl * 8 + xcd;
  } else {
    nt = id % ntiles8;
    const int rest = id / ntiles8;
    s = rest % S;
    mt = rest / S;
  }
  if (nt >= ntiles) return;
  const int M = Mdev ? min(*Mdev, Mcap) : Mcap;
  const int m0 = mt * MT;
  if (m0 >= M) return;
  const int n0 = nt * NT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int C = K >> 6;
  const int c_beg = (int)((int64_t)s * C / S), c_end = (int)((int64_t)(s + 1) * C / S);
  const int n = c_end - c_beg;
  const int64_t KS32 = K >> 5;
  // this wave's A blocks of a chunk: q = wave + 4 u, row block q / 2, k step q % 2
  const int last_blk = (M - 1) >> 4;
  const bf16_t* abase[AB];
#pragma unroll
  for (int u = 0; u < AB; ++u) {
    const int q = wave + 4 * u;
    abase[u] = A + ((int64_t)min(m0 / 16 + q / 2, last_blk) * KS32 + (q & 1)) * 512 + lane * 8;
  }
  const bf16_t* wbase[NBW];
#pragma unroll
  for (int j = 0; j < NBW; ++j) wbase[j] = W + (int64_t)(n0 / 16 + wave * NBW + j) * KS32 * 512 + lane * 8;

  RmsPre rpre;  // folded RMSNorm: this thread's share of row m0 + t / (256 / MT)
  if constexpr (EPI == EPI_RELU2) {
    if (e.rms_in != nullptr) rms_load<16 * MB>(rpre, e, m0, M);
  }
  QkvPre qpre[(MB + 1) / 2];  // EPI_QKV: cache row / position of this thread's token in each 32-row pass
  if constexpr (EPI == EPI_QKV) {
#pragma unroll
    for (int p = 0; p < MB / 2; ++p) qkv_pre_row(e.qkv, m0 + 32 * p + (threadIdx.x >> 3), M, nt, qpre[p]);
  }
  // EPI_SOFTCAP draw noise: the row's round counter loads ahead of the
  // operands, so waiting for it does not wait for them
  VpNoise<MB, NBW> nz;
  nz.ok = false;
  int vp_rnd = 0;
  if constexpr (EPI == EPI_SOFTCAP && MB == 2) {
    const int mrow = m0 + (threadIdx.x >> 3);
    if (vp_noise_wanted<MB, NBW>(e) && mrow < M) vp_rnd = e.vp_round[mrow];
  }
  f32x4 acc[MB][NBW];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NBW; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (n > 0) {
    v4u wr[NS][NBW][2], ar[NS][AB];
#define LA_LOAD(slot, i)                                                              \
  {                                                                                   \
    const int c_ = c_beg + min((i), n - 1);                                           \
    _Pragma("unroll") for (int j = 0; j < NBW; ++j)                                   \
      _Pragma("unroll") for (int ks = 0; ks < 2; ++ks)                                \
        wr[slot][j][ks] = EPI == EPI_SOFTCAP ? LM_LD((const v4u*)(wbase[j] + (2 * c_ + ks) * 512)) \
                                             : W_LD((const v4u*)(wbase[j] + (2 * c_ + ks) * 512));   \
    _Pragma("unroll") for (int u = 0; u < AB; ++u)                                    \
      ar[slot][u] = *(const v4u*)(abase[u] + (int64_t)c_ * 1024);                     \
  }
#define LA_STAGE_A(slot, buf)                                                         \
  {                                                                                   \
    _Pragma("unroll") for (int u = 0; u < AB; ++u)                                    \
      As[buf][wave + 4 * u][lane] = __builtin_bit_cast(uint4, ar[slot][u]);           \
  }
#pragma unroll
    for (int p = 0; p < NS; ++p) LA_LOAD(p, p);
    if constexpr (EPI == EPI_SOFTCAP && MB == 2) vp_noise<MB, NBW>(e, m0, n0, vp_rnd, nz);
    LA_STAGE_A(0, 0);
    __syncthreads();
    for (int i0 = 0; i0 < n; i0 += NS) {
#pragma unroll
      for (int p = 0; p < NS; ++p) {
        const int i = i0 + p;
        const int buf = i & 1;
        if (i < n) {
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
              const v4u a = __builtin_bit_cast(v4u, As[buf][2 * mb + ks][lane]);
#pragma unroll
              for (int j = 0; j < NBW; ++j) acc[mb][j] = mfma16(a, wr[p][j][ks], acc[mb][j]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // next chunk's A into the other LDS buffer (its last reader was
        // chunk i - 1, finished before the previous barrier), then refill
        // the freed ring slots
        LA_STAGE_A((p + 1) % NS, buf ^ 1);
        __builtin_amdgcn_sched_barrier(0);
        LA_LOAD(p, i + NS);
        __syncthreads();
      }
    }
#undef LA_LOAD
#undef LA_STAGE_A
  }

  tile_epilogue<MB, NBW, EPI, true>(e, acc, rpre, qpre, m0, n0, nt, s, M, K, &nz);
}

// bf16 MFMA GEMM for verify-size row counts with both operands staged in an
// LDS ring by direct global-to-LDS loads.
//
// Same tile and column split as k_gemm_la (MT = 16 MB rows, NT = 64 NBW
// columns, each wave owns 16 NBW columns), but the activation blocks and the
// wave's own weight blocks of a 64-wide k chunk go straight from global
// memory into one of four LDS stages (no registers held by loads in flight):
// while chunk i computes, chunks i+1 and i+2 are loading. Each stage is its
// own LDS object and the loop is unrolled over the four, so the compiler can
// tell a stage's reads from the loads into the others and waits only for the
// chunk it needs (vmcnt(two chunks' loads)), then a plain barrier makes every
// wave's part of the stage visible. The stage refilled at step i is the one
// read at step i-1, which every wave has finished by the barrier of step i.
// Grid and tile order as in k_gemm_la.
template <int MB, int NBW>
struct DmaStage {
  uint4 a[2 * MB][64];
  uint4 w[4][2 * NBW][64];
};
template <int MB, int NBW, int EPI>
__global__ __launch_bounds__(256) void k_gemm_dma(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W,
                                                  int Mcap, const int* __restrict__ Mdev, int N, int K, int ntiles,
                                                  int mtiles, int mfast, Epi e) {
  constexpr int WAVES = 4, AB = 2 * MB, NSTG = 4;
  static_assert(AB % WAVES == 0, "the A blocks of a chunk split evenly over the waves");
  __shared__ DmaStage<MB, NBW> s0, s1, s2, s3;
  const int id = blockIdx.x;
  const int ntiles8 = (ntiles + 7) & ~7;
  int nt, mt;
  if (mfast) {
    const int xcd = id & 7, loc = id >> 3;
    const int nl = loc / mtiles;
    mt = loc - nl * mtiles;
    nt = nl * 8 + xcd;
  } else {
    nt = id % ntiles8;
    mt = id / ntiles8;
  }
  if (nt >= ntiles) return;
  const int M = Mdev ? min(*Mdev, Mcap) : Mcap;
  const int m0 = mt * 16 * MB;
  if (m0 >= M) return;
  const int n0 = nt * 64 * NBW;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t KS32 = K >> 5;
  const int C = K >> 6;
  const int last_blk = (M - 1) >> 4;
  const bf16_t* wbase = W + ((int64_t)(n0 / 16 + wave * NBW)) * KS32 * 512 + lane * 8;
  const bf16_t* abase[AB / WAVES];
#pragma unroll
  for (int u = 0; u < AB / WAVES; ++u) {
    const int q = wave + WAVES * u;  // row block q / 2, k step q % 2
    abase[u] = A + ((int64_t)min(m0 / 16 + (q >> 1), last_blk) * KS32 + (q & 1)) * 512 + lane * 8;
  }
  RmsPre rpre;  // folded RMSNorm: this thread's share of row m0 + t / (256 / MT)
  if constexpr (EPI == EPI_RELU2) {
    if (e.rms_in != nullptr) rms_load<16 * MB>(rpre, e, m0, M);
  }
  QkvPre qpre[(MB + 1) / 2];  // unused: the fused QKV epilogue runs on k_gemm_la and k_gemm_big
  f32x4 acc[MB][NBW];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NBW; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // loads per chunk and wave: 2 NBW weight blocks + AB / WAVES activation blocks
  constexpr int PER = 2 * NBW + AB / WAVES;
  constexpr int NV = PER * (NSTG - 2);
  static_assert(NV < 64, "vmcnt range");
#define DMA_ISSUE(S, c_)                                                                             \
  {                                                                                                  \
    const int c = min((c_), C - 1); /* past the end: harmless re-reads into an unread stage */       \
    _Pragma("unroll") for (int j = 0; j < NBW; ++j)                                                  \
      _Pragma("unroll") for (int ks = 0; ks < 2; ++ks)                                               \
        __builtin_amdgcn_global_load_lds((const void*)(wbase + ((int64_t)j * KS32 + 2 * c + ks) * 512), \
                                         (__attribute__((address_space(3))) void*)&S.w[wave][2 * j + ks][0], 16, 0, 0); \
    _Pragma("unroll") for (int u = 0; u < AB / WAVES; ++u)                                           \
      __builtin_amdgcn_global_load_lds((const void*)(abase[u] + (int64_t)c * 1024),                  \
                                       (__attribute__((address_space(3))) void*)&S.a[wave + WAVES * u][0], 16, 0, 0); \
  }
#define DMA_STEP(S, SN, i_)                                                                          \
  {                                                                                                  \
    __builtin_amdgcn_s_waitcnt((NV & 15) | ((NV >> 4) << 14) | (7 << 4) | (15 << 8));                \
    __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                         \
    __builtin_amdgcn_sched_barrier(0);                                                               \
    __builtin_amdgcn_s_barrier();                                                                    \
    __builtin_amdgcn_sched_barrier(0);                                                               \
    __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                         \
    _Pragma("unroll") for (int ks = 0; ks < 2; ++ks) {                                               \
      v4u w[NBW];                                                                                    \
      _Pragma("unroll") for (int j = 0; j < NBW; ++j) w[j] = __builtin_bit_cast(v4u, S.w[wave][2 * j + ks][lane]); \
      _Pragma("unroll") for (int mb = 0; mb < MB; ++mb) {                                            \
        const v4u a = __builtin_bit_cast(v4u, S.a[2 * mb + ks][lane]);                               \
        _Pragma("unroll") for (int j = 0; j < NBW; ++j) acc[mb][j] = mfma16(a, w[j], acc[mb][j]);    \
      }                                                                                              \
    }                                                                                                \
    DMA_ISSUE(SN, (i_) + NSTG - 1);                                                                  \
  }
  DMA_ISSUE(s0, 0);
  DMA_ISSUE(s1, 1);
  DMA_ISSUE(s2, 2);
  int i = 0;
  for (; i + 3 < C; i += 4) {
    DMA_STEP(s0, s3, i);
    DMA_STEP(s1, s0, i + 1);
    DMA_STEP(s2, s1, i + 2);
    DMA_STEP(s3, s2, i + 3);
  }
  if (i < C) DMA_STEP(s0, s3, i);
  if (i + 1 < C) DMA_STEP(s1, s0, i + 1);
  if (i + 2 < C) DMA_STEP(s2, s1, i + 2);
#undef DMA_STEP
#undef DMA_ISSUE
  __builtin_amdgcn_s_waitcnt(0);  // no direct load outlives the workgroup's LDS
  __syncthreads();                // the epilogue may reuse LDS
  tile_epilogue<MB, NBW, EPI>(e, acc, rpre, qpre, m0, n0, nt, 0, M, K);
}

// bf16 MFMA GEMM for verify-size row counts with every operand block in a
// deep LDS ring fed by direct global-to-LDS loads.
//
// A workgroup owns an MT x NT tile (MT = 16 MB rows, NT = 16 NB columns) of
// one K split; its four waves form a WM x (4 / WM) grid over (row blocks,
// column blocks). Per 64-wide k chunk the tile needs 2 MB activation and
// 2 NB weight blocks of 1 KB (fragment order); they go straight into stage
// chunk % NSTG of the ring, PER per wave, with no registers held by loads in
// flight. Step i waits until the wave's own loads of chunk i have landed
// (vmcnt: the NSTG - 2 later chunks may still be in flight), meets the other
// waves at a barrier (so every wave's part of the stage is visible and every
// wave has finished reading stage i - 1), refills stage i - 1 with chunk
// i + NSTG - 1, then reads its fragments of stage i and runs its MFMAs.
// Each stage is its own LDS object and the loop is unrolled over the ring,
// so the compiler can tell a stage's reads from the loads into the others.
// Against the register-staged kernels this keeps NSTG - 1 chunks in flight
// per workgroup instead of one or two: at the cfg4 verify MLP c_proj shape
// (224 rows, N 1536, K 6144, 64 x 96 tiles, K split 4: 256 workgroups) it
// takes 13.4-13.8 us against 15.4 us for the 32 x 64 split-3 tiles of
// k_gemm_ks (weights cycled from HBM). Measured limits: with the weights
// resident in L2 its loads alone run at ~120 GB/s per CU (the L2-resident
// read ceiling), and its LDS traffic (stage writes plus fragment reads,
// 3x the global bytes at a 2 x 2 wave grid) then bounds it; streaming the
// weights from HBM adds ~3 us per launch that the ring depth does not hide.
// Grid: N tile fastest (tile n on XCD n % 8: the M tiles and splits of one
// weight slab share that XCD's L2), then split, then M tile; tiles past the
// device row count exit at once.
template <int TOT>
struct RingStage {
  uint4 blk[TOT][64];
};
template <int MB, int NB, int NSTG, int WM, int EPI>
__global__ __launch_bounds__(256) void k_gemm_ring(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W,
                                                   int Mcap, const int* __restrict__ Mdev, int N, int K, int ntiles,
                                                   int S, Epi e) {
  constexpr int WN = 4 / WM, MBW = MB / WM, NBW = NB / WN;
  static_assert(MB % WM == 0 && NB % WN == 0, "wave grid");
  constexpr int TOT = 2 * MB + 2 * NB, PER = (TOT + 3) / 4, NV = PER * (NSTG - 2);
  static_assert(NV < 64 && NSTG >= 3 && NSTG <= 8, "ring depth / vmcnt range");
  __shared__ RingStage<TOT> s0, s1, s2, s3, s4, s5, s6, s7;  // the first NSTG are used
  const int id = blockIdx.x;
  const int ntiles8 = (ntiles + 7) & ~7;
  const int nt = id % ntiles8;
  const int rest = id / ntiles8;
  const int s = rest % S, mt = rest / S;
  if (nt >= ntiles) return;
  const int M = Mdev ? min(*Mdev, Mcap) : Mcap;
  const int m0 = mt * 16 * MB;
  if (m0 >= M) return;
  const int n0 = nt * 16 * NB;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int r = lane & 15, g = lane >> 4;
  const int C = K >> 6;
  const int c_beg = (int)((int64_t)s * C / S), c_end = (int)((int64_t)(s + 1) * C / S);
  const int n = c_end - c_beg;
  const int64_t KS32 = K >> 5;
  const int last_blk = (M - 1) >> 4;
  // this wave's blocks of a chunk: q < 2 MB activation row block q / 2, else
  // weight column block (q - 2 MB) / 2; k step q % 2. A wave with fewer than
  // PER distinct blocks repeats the last one (the same bytes into the same
  // LDS slot, harmless).
  const bf16_t* src[PER];
  int dst[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int q = min(wave + 4 * u, TOT - 1);
    dst[u] = q;
    if (q < 2 * MB) {
      src[u] = A + ((int64_t)min(m0 / 16 + (q >> 1), last_blk) * KS32 + (q & 1)) * 512 + lane * 8;
    } else {
      const int j2 = q - 2 * MB;
      src[u] = W + ((int64_t)(n0 / 16 + (j2 >> 1)) * KS32 + (j2 & 1)) * 512 + lane * 8;
    }
  }
  RmsPre rpre;  // folded RMSNorm: this thread's share of row m0 + t / (256 / MT)
  if constexpr (EPI == EPI_RELU2) {
    if (e.rms_in != nullptr) rms_load<16 * MB>(rpre, e, m0, M);
  }
  f32x4 acc[MBW][NBW];
#pragma unroll
  for (int i = 0; i < MBW; ++i)
#pragma unroll
    for (int j = 0; j < NBW; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#define RING_STG(k) (k == 0 ? s0 : k == 1 ? s1 : k == 2 ? s2 : k == 3 ? s3 : k == 4 ? s4 : k == 5 ? s5 : k == 6 ? s6 : s7)
#define RING_ISSUE(k, c_)                                                                                  \
  {                                                                                                        \
    const int64_t cc_ = (int64_t)(c_beg + min((c_), n - 1)) * 1024; /* past the end: harmless re-reads */  \
    _Pragma("unroll") for (int u = 0; u < PER; ++u)                                                        \
      __builtin_amdgcn_global_load_lds((const void*)(src[u] + cc_),                                        \
                                       (__attribute__((address_space(3))) void*)&RING_STG(k).blk[dst[u]][0], \
                                       16, 0, 0);                                                          \
  }
#define RING_STEP(k, i_)                                                                                   \
  {                                                                                                        \
    __builtin_amdgcn_sched_barrier(0);                                                                     \
    __builtin_amdgcn_s_waitcnt((NV & 15) | ((NV >> 4) << 14) | (7 << 4) | (15 << 8));                      \
    __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                               \
    __builtin_amdgcn_sched_barrier(0);                                                                     \
    __builtin_amdgcn_s_barrier();                                                                          \
    __builtin_amdgcn_sched_barrier(0);                                                                     \
    __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                               \
    RING_ISSUE(((k) + NSTG - 1) % NSTG, (i_) + NSTG - 1);                                                  \
    _Pragma("unroll") for (int ks = 0; ks < 2; ++ks) {                                                     \
      v4u af[MBW], wf[NBW];                                                                                \
      _Pragma("unroll") for (int i = 0; i < MBW; ++i)                                                      \
        af[i] = __builtin_bit_cast(v4u, RING_STG(k).blk[2 * (wm * MBW + i) + ks][lane]);                   \
      _Pragma("unroll") for (int j = 0; j < NBW; ++j)                                                      \
        wf[j] = __builtin_bit_cast(v4u, RING_STG(k).blk[2 * MB + 2 * (wn * NBW + j) + ks][lane]);          \
      _Pragma("unroll") for (int i = 0; i < MBW; ++i)                                                      \
        _Pragma("unroll") for (int j = 0; j < NBW; ++j) acc[i][j] = mfma16(af[i], wf[j], acc[i][j]);       \
    }                                                                                                      \
  }
  if (n > 0) {
#pragma unroll
    for (int c = 0; c < NSTG - 1; ++c) RING_ISSUE(c, c);
    int i = 0;
    for (; i + NSTG <= n; i += NSTG) {
      RING_STEP(0, i);
      RING_STEP(1, i + 1);
      RING_STEP(2, i + 2);
      if (NSTG > 3) RING_STEP(3 % NSTG, i + 3);
      if (NSTG > 4) RING_STEP(4 % NSTG, i + 4);
      if (NSTG > 5) RING_STEP(5 % NSTG, i + 5);
      if (NSTG > 6) RING_STEP(6 % NSTG, i + 6);
      if (NSTG > 7) RING_STEP(7 % NSTG, i + 7);
    }
    // the last n - i < NSTG chunks sit in stages 0 .. n - i - 1
    if (i < n) RING_STEP(0, i);
    if (i + 1 < n) RING_STEP(1, i + 1);
    if (NSTG > 3 && i + 2 < n) RING_STEP(2, i + 2);
    if (NSTG > 4 && i + 3 < n) RING_STEP(3 % NSTG, i + 3);
    if (NSTG > 5 && i + 4 < n) RING_STEP(4 % NSTG, i + 4);
    if (NSTG > 6 && i + 5 < n) RING_STEP(5 % NSTG, i + 5);
    if (NSTG > 7 && i + 6 < n) RING_STEP(6 % NSTG, i + 6);
  }
#undef RING_STEP
#undef RING_ISSUE
#undef RING_STG
  __builtin_amdgcn_s_waitcnt(0);  // no direct load outlives the workgroup's LDS
  if constexpr (EPI == EPI_RELU2 || EPI == EPI_ADD) {
    // ReLU^2 and the residual add go through the row-major epilogue (the
    // folded RMSNorm works on whole row segments): stage the tile in LDS
    constexpr int MT = 16 * MB, NT = 16 * NB, OPT = MT * NT / 256, TPR = NT / OPT;
    static_assert(OPT >= 1 && NT % OPT == 0, "epilogue tiling");
    __shared__ float red[MT][NT + 4];
#pragma unroll
    for (int mb = 0; mb < MBW; ++mb)
#pragma unroll
      for (int j = 0; j < NBW; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[16 * (wm * MBW + mb) + 4 * g + i][16 * (wn * NBW + j) + r] = acc[mb][j][i];
    __syncthreads();
    const int t = threadIdx.x;
    const int row = t / TPR, col0 = (t - row * TPR) * OPT;
    float v[OPT];
#pragma unroll
    for (int c = 0; c < OPT; ++c) v[c] = red[row][col0 + c];
    row_epilogue<EPI, MT, NT>(e, v, row, col0, m0, n0, nt, s, M, K, rpre);
  } else {
    Epi ee = e;
    ee.split = s;
#pragma unroll
    for (int mb = 0; mb < MBW; ++mb)
#pragma unroll
      for (int j = 0; j < NBW; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = m0 + 16 * (wm * MBW + mb) + 4 * g + i;
          if (m < M) epi_apply<EPI, true>(ee, m, n0 + 16 * (wn * NBW + j) + r, acc[mb][j][i]);
        }
  }
}

// bf16 MFMA GEMM for prefill-size row counts (M >= FC_BIG_M, N % 256 == 0,
// K % 128 == 0).
//
// A workgroup owns a 256 x 256 output tile; each of its four waves owns a
// 128 x 128 quadrant as 4 x 4 blocks of 32 x 32 (the 32x32x16 MFMA: with
// one wave per SIMD it keeps the matrix unit ~86% busy, where 16x16x32
// chains reach about half), 256 accumulators per lane. Per 32-wide k step
// the tile needs 16 activation and 16 weight blocks of 1 KB (16 rows x 32 k,
// fragment order); they go straight from global memory into one of four
// 32 KB LDS stages by direct loads, 8 per wave. The 32x32x16 operand of
// lane l is row l % 32, k 8 (l / 32) .. +7 of a 16-k half: 16 bytes that sit
// in 16-row block (l % 32) / 16 at lane slot l % 16 + 16 (2 half + l / 32),
// so the stored layout feeds it unchanged.
//
// Per step i: wait until stage i+1 has landed (own loads: vmcnt(16), the two
// later stages may still be in flight) and every wave has finished reading
// stage i into registers (lgkmcnt(0)); one barrier; start reading stage i+1
// into the other fragment set; refill stage i with chunk i+4; then the 32
// MFMAs of step i run on fragments already in registers.
//
// The MFMA takes the weight block as its first operand, so a lane's result
// is row m0 + l % 32 and, per group of four registers, four consecutive
// columns: fp32 outputs are written as float4, and the bf16 fragment-order
// output (ReLU^2, the next GEMM's operand) goes through a 32 x 32 LDS
// transpose per wave (8-byte writes, 16-byte reads).
//
// Tile order: tiles are grouped by 4 M tiles (N tile slower within a group)
// and dealt to the eight XCDs in contiguous ranges, so the ~32 workgroups
// an XCD runs at once cover about 4 M tiles x 8 N tiles and share their
// operand slabs in that XCD's L2.
#ifndef FC_BIG_M
#define FC_BIG_M 1024
#endif
#ifndef FC_BIG_MIN_TILES
#define FC_BIG_MIN_TILES 224
#endif
// Wide outputs (the lm_head, N >= 16384) take the 256 x 256 tiles from this
// many rows: the cfg4 verify head (224 rows, 256 tiles) runs 78.7 us on them
// against 92.7 us on the LDS-shared 128 x 128 tiles (kernel trace); the
// round gains ~3 us of it (4.814-4.818 vs 4.817-4.820 ms, alternating builds).
#ifndef FC_BIG_HEAD_M
#define FC_BIG_HEAD_M 200
#endif
template <int NB>
struct BigStage {
  uint4 a[16][64];
  uint4 w[4 * NB][64];
};
template <int EPI>
__device__ __forceinline__ void big_store4(const Epi& e, int m, int n, float v0, float v1, float v2, float v3,
                                           int split) {
  if constexpr (EPI == EPI_STORE) {
    *(float4*)((float*)e.out + (int64_t)m * e.ldo + n) = float4{v0, v1, v2, v3};
  } else if constexpr (EPI == EPI_ADD) {
    float4* o = (float4*)((float*)e.out + (int64_t)m * e.ldo + n);
    const float4 x = *o;
    *o = float4{x.x + v0, x.y + v1, x.z + v2, x.w + v3};
  } else if constexpr (EPI == EPI_MLPOUT) {
    const int64_t i = (int64_t)m * e.ldo + n;
    float4* xp = (float4*)((float*)e.out + i);
    const float4 x = *xp;
    const float4 t = float4{x.x + v0, x.y + v1, x.z + v2, x.w + v3};  // engine.py:161
    float4 xb = float4{0.f, 0.f, 0.f, 0.f};
    if (e.capture) {                                                   // engine.py:164
      *(float4*)(e.xb + i) = t;
      xb = t;
    } else if (e.last) {
      xb = *(const float4*)(e.xb + i);
    }
    if (e.last) {                                                      // engine.py:166
      *xp = float4{t.x - e.lb * xb.x, t.y - e.lb * xb.y, t.z - e.lb * xb.z, t.w - e.lb * xb.w};
    } else {                                                           // engine.py:94
      const float4 x0 = *(const float4*)(e.x0 + i);
      *xp = float4{e.r * t.x + e.a * x0.x, e.r * t.y + e.a * x0.y, e.r * t.z + e.a * x0.z, e.r * t.w + e.a * x0.w};
    }
  } else if constexpr (EPI == EPI_PARTIAL) {  // split-K partial, finished by the next RMSNorm
    *(float4*)(e.part + ((int64_t)split * e.part_rows + m) * e.ldo + n) = float4{v0, v1, v2, v3};
  } else if constexpr (EPI == EPI_SOFTCAP) {  // logits row (m / n_out, m % n_out), columns past V dropped
    const int b = m / e.n_out, rr = m - b * e.n_out;
    float* o = (float*)e.out + (int64_t)b * e.row_stride + (int64_t)rr * e.V + n;
    const float t0 = softcap15_fast(v0), t1 = softcap15_fast(v1);
    const float t2 = softcap15_fast(v2), t3 = softcap15_fast(v3);
    if (n + 3 < e.V && (((uintptr_t)o) & 15) == 0) {
      *(float4*)o = float4{t0, t1, t2, t3};
    } else {
      if (n < e.V) o[0] = t0;
      if (n + 1 < e.V) o[1] = t1;
      if (n + 2 < e.V) o[2] = t2;
      if (n + 3 < e.V) o[3] = t3;
    }
  } else {
    epi_apply<EPI, true>(e, m, n, v0);
    epi_apply<EPI, true>(e, m, n + 1, v1);
    epi_apply<EPI, true>(e, m, n + 2, v2);
    epi_apply<EPI, true>(e, m, n + 3, v3);
  }
}
template <int EPI, int NB>
__global__ __launch_bounds__(256) void k_gemm_big(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W,
                                                  int Mcap, const int* __restrict__ Mdev, int N, int K, int ntiles,
                                                  int mtiles, int per_xcd, int S, Epi e) {
  // NB 32-column blocks per wave: tile 256 x 64 NB (NB = 4: 256 x 256; NB = 3: 256 x 192)
  constexpr int NSTG = 4, GM = 4, NT = 64 * NB;
  static_assert(NB == 3 || NB == 4, "tile widths 192 and 256");
  static_assert(EPI != EPI_QKV || NB == 4, "the QKV epilogue needs one head (128 columns) per wave");
  __shared__ BigStage<NB> s0, s1, s2, s3;
  // tile of this workgroup. Unsplit: XCD id % 8 takes grouped tiles
  // [x per_xcd, (x + 1) per_xcd). Split 8 ways in K (EPI_PARTIAL): XCD x
  // takes split x, whose workgroups share its A and W slabs in that XCD's L2,
  // M tile slowest, so the live tiles (below the device row count) come
  // first and the plan keeps them within the XCD's 32 CUs.
  int sp, nt, mt;
  if (S == 8) {
    sp = blockIdx.x & 7;
    const int j = blockIdx.x >> 3;
    if (j >= ntiles * mtiles) return;
    mt = j / ntiles;
    nt = j - mt * ntiles;
  } else {
    const int t = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if ((int)(blockIdx.x >> 3) >= per_xcd || t >= ntiles * mtiles) return;
    const int grp = t / (GM * ntiles), rr = t - grp * GM * ntiles;
    const int gm = min(GM, mtiles - grp * GM);
    nt = rr / gm;
    mt = grp * GM + rr % gm;
    sp = 0;
  }
  const int M = Mdev ? min(*Mdev, Mcap) : Mcap;
  const int m0 = mt * 256;
  if (m0 >= M) return;
  const int n0 = nt * NT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t KS32 = K >> 5;
  // this split's 32-deep k steps [c0, c0 + C); the host makes C a multiple of 4
  const int c0 = (int)(sp * KS32 / S), C = (int)((sp + 1) * KS32 / S) - c0;
  const int last_blk = (M - 1) >> 4;
  // this wave's loads: activation row blocks 4 wave .. +3 and weight column blocks NB wave .. +NB-1
  const bf16_t* ab[4];
  const bf16_t* wb[NB];
#pragma unroll
  for (int u = 0; u < 4; ++u)
    ab[u] = A + ((int64_t)min(m0 / 16 + 4 * wave + u, last_blk) * KS32 + c0) * 512 + lane * 8;
#pragma unroll
  for (int u = 0; u < NB; ++u) wb[u] = W + ((int64_t)(n0 / 16 + NB * wave + u) * KS32 + c0) * 512 + lane * 8;
  // this lane's 32x32x16 operand slot: 16-row block offset and lane slot (half 0; +32 for half 1)
  const int sub = (lane & 31) >> 4, slot = (lane & 15) + 16 * (lane >> 5);
  f32x16 acc[4][NB];
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int q = 0; q < NB; ++q)
#pragma unroll
      for (int x = 0; x < 16; ++x) acc[p][q][x] = 0.f;
  constexpr int NV = (4 + NB) * (NSTG - 2);
  static_assert(NV < 64, "vmcnt range");
#define BIG_ISSUE(S, c_)                                                                                      \
  {                                                                                                           \
    const int c = min((c_), C - 1); /* past the end: harmless re-reads into an unread stage */                \
    _Pragma("unroll") for (int u = 0; u < 4; ++u)                                                             \
      __builtin_amdgcn_global_load_lds((const void*)(ab[u] + (int64_t)c * 512),                              \
                                       (__attribute__((address_space(3))) void*)&S.a[4 * wave + u][0], 16, 0, 0); \
    _Pragma("unroll") for (int u = 0; u < NB; ++u)                                                            \
      __builtin_amdgcn_global_load_lds((const void*)(wb[u] + (int64_t)c * 512),                              \
                                       (__attribute__((address_space(3))) void*)&S.w[NB * wave + u][0], 16, 0,   \
                                       EPI == EPI_SOFTCAP && FC_BIG_LM_NT ? 2 : 0);                          \
  }
#define BIG_SYNC(NVW)                                                                                         \
  {                                                                                                           \
    __builtin_amdgcn_sched_barrier(0); /* the wait must not rise above the previous step's MFMAs */           \
    __builtin_amdgcn_s_waitcnt(((NVW) & 15) | (((NVW) >> 4) << 14) | (7 << 4) | (0 << 8));                  \
    __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                                  \
    __builtin_amdgcn_sched_barrier(0);                                                                        \
    __builtin_amdgcn_s_barrier();                                                                             \
    __builtin_amdgcn_sched_barrier(0);                                                                        \
    __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                                  \
  }
  // fragments of one k step: [half][32-row / 32-column block]
#define BIG_READ(S, WF, AF)                                                                                   \
  {                                                                                                           \
    _Pragma("unroll") for (int h = 0; h < 2; ++h) {                                                           \
      _Pragma("unroll") for (int b = 0; b < NB; ++b)                                                          \
        WF[h][b] = __builtin_bit_cast(v4u, S.w[2 * NB * wn + 2 * b + sub][slot + 32 * h]);                    \
      _Pragma("unroll") for (int b = 0; b < 4; ++b)                                                           \
        AF[h][b] = __builtin_bit_cast(v4u, S.a[8 * wm + 2 * b + sub][slot + 32 * h]);                         \
    }                                                                                                         \
  }
#define BIG_MMA(WF, AF)                                                                                       \
  {                                                                                                           \
    _Pragma("unroll") for (int h = 0; h < 2; ++h)                                                             \
      _Pragma("unroll") for (int p = 0; p < 4; ++p)                                                           \
        _Pragma("unroll") for (int q = 0; q < NB; ++q) acc[p][q] = mfma32(WF[h][q], AF[h][p], acc[p][q]);     \
  }
  // step i: SN = stage of chunk i + 1 (read now), SI = stage of chunk i (refilled with chunk i + 4)
#define BIG_STEP(SI, SN, WFC, AFC, WFN, AFN, i_)                                                              \
  {                                                                                                           \
    BIG_SYNC(NV);                                                                                             \
    BIG_READ(SN, WFN, AFN);                                                                                   \
    BIG_ISSUE(SI, (i_) + NSTG);                                                                               \
    BIG_MMA(WFC, AFC);                                                                                        \
  }
  v4u wf0[2][NB], af0[2][4], wf1[2][NB], af1[2][4];
  BIG_ISSUE(s0, 0);
  BIG_ISSUE(s1, 1);
  BIG_ISSUE(s2, 2);
  BIG_ISSUE(s3, 3);
  BIG_SYNC(3 * (4 + NB));  // chunk 0 landed: at most the 3 later chunks' loads outstanding
  BIG_READ(s0, wf0, af0);
  // C % 4 == 0 (K % 128 == 0): 4-step groups, the last one ends without a read
  int i = 0;
  for (; i + 4 < C; i += 4) {
    BIG_STEP(s0, s1, wf0, af0, wf1, af1, i);
    BIG_STEP(s1, s2, wf1, af1, wf0, af0, i + 1);
    BIG_STEP(s2, s3, wf0, af0, wf1, af1, i + 2);
    BIG_STEP(s3, s0, wf1, af1, wf0, af0, i + 3);
  }
  BIG_STEP(s0, s1, wf0, af0, wf1, af1, i);
  BIG_STEP(s1, s2, wf1, af1, wf0, af0, i + 1);
  BIG_STEP(s2, s3, wf0, af0, wf1, af1, i + 2);
  BIG_MMA(wf1, af1);
#undef BIG_STEP
#undef BIG_MMA
#undef BIG_READ
#undef BIG_SYNC
#undef BIG_ISSUE
  __builtin_amdgcn_s_waitcnt(0);  // no direct load outlives the workgroup's LDS
  __syncthreads();                // stage s0 becomes the epilogue's scratch
  // lane l holds row 32 p + l % 32 of the quadrant; register 4 j + x holds
  // column 32 q + 8 j + 4 (l / 32) + x
  const int rl = lane & 31, ch = 4 * (lane >> 5);
  if constexpr (EPI == EPI_QKV) {
    // the quadrant is one head slot (128 columns) for 128 tokens: per 32
    // tokens, stage the rows in this wave's own LDS stage (fp32), then eight
    // lanes per token finish RoPE / QK-norm / VE gate / KV append
    BigStage<NB>* mine = wave == 0 ? &s0 : wave == 1 ? &s1 : wave == 2 ? &s2 : &s3;
    float(*T)[128 + 4] = (float(*)[128 + 4])mine;
    const int hh = (n0 + 128 * wn) >> 7;
    const int mq = m0 + 128 * wm + (lane >> 3);  // this lane's token in group p, step it: mq + 32 p + 8 it
    int rb[4][4], rp[4][4], rt[4][4];             // their cache rows / positions / ids, loaded together
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        QkvPre r;
        qkv_pre_row(e.qkv, mq + 32 * p + 8 * it, M, hh, r);
        rb[p][it] = r.b;
        rp[p][it] = r.pos;
        rt[p][it] = r.tok;
      }
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      QkvPre pre[4];  // table / value-embedding loads of the group's 4 tokens, in flight while it is staged
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        pre[it].b = rb[p][it];
        pre[it].pos = rp[p][it];
        pre[it].tok = rt[p][it];
        qkv_pre_tab(e.qkv, mq + 32 * p + 8 * it, M, hh, lane & 7, pre[it]);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *(float4*)&T[rl][32 * q + 8 * j + ch] =
              float4{acc[p][q][4 * j], acc[p][q][4 * j + 1], acc[p][q][4 * j + 2], acc[p][q][4 * j + 3]};
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int tt = 8 * it + (lane >> 3);
        qkv_finish(e.qkv, T[tt], m0 + 128 * wm + 32 * p + tt, M, hh, lane & 7, pre[it]);
      }
      __builtin_amdgcn_wave_barrier();
    }
  } else if constexpr (EPI == EPI_RELU2) {
    // bf16 fragment order: per 32 x 32 block, lane l writes row l % 32,
    // columns 8 j + 4 (l / 32) .. +3 into a 32 x 80 B scratch; then per
    // 16-row half, lane L reads row L % 16, columns 8 (L / 16) .. +7
    char* scr = (char*)&s0 + wave * 32 * 80;
    bf16_t* out = (bf16_t*)e.out;
    const int KB = e.ldo >> 5;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
#pragma unroll
      for (int q = 0; q < NB; ++q) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          uint32_t pk[2];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const float x0 = fmaxf(acc[p][q][4 * j + 2 * hh], 0.f), x1 = fmaxf(acc[p][q][4 * j + 2 * hh + 1], 0.f);
            pk[hh] = (uint32_t)f2bf(x0 * x0) | ((uint32_t)f2bf(x1 * x1) << 16);
          }
          *(uint2*)(scr + rl * 80 + (8 * j + ch) * 2) = uint2{pk[0], pk[1]};
        }
        const int kb = (n0 + 32 * NB * wn + 32 * q) >> 5;
#pragma unroll
        for (int hs = 0; hs < 2; ++hs) {
          const uint4 val = *(const uint4*)(scr + (16 * hs + (lane & 15)) * 80 + 16 * (lane >> 4));
          const int rb = (m0 + 128 * wm + 32 * p + 16 * hs) >> 4;
          if (16 * rb < M) *(uint4*)(out + ((int64_t)rb * KB + kb) * 512 + lane * 8) = val;
        }
      }
    }
  } else {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int m = m0 + 128 * wm + 32 * p + rl;
      if (m < M) {
#pragma unroll
        for (int q = 0; q < NB; ++q)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            big_store4<EPI>(e, m, n0 + 32 * NB * wn + 32 * q + 8 * j + ch, acc[p][q][4 * j], acc[p][q][4 * j + 1],
                            acc[p][q][4 * j + 2], acc[p][q][4 * j + 3], sp);
      }
    }
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
static void launch_gemv_mb(const void* A, const void* W, int M, const int* Mdev, int N, int K, const Epi& e,
                           hipStream_t s) {
  const dim3 grid((N + 15) / 16, (M + MB - 1) / MB);
  FC_EPI_SWITCH(e.mode, hipLaunchKernelGGL((k_gemv<T, MB, E>), grid, dim3(256), 0, s, (const T*)A, (const T*)W, M,
                                           Mdev, N, K, e));
}
template <typename T>
static void launch_gemv(const void* A, const void* W, int M, const int* Mdev, int N, int K, const Epi& e,
                        hipStream_t s) {
  if (M <= 1) launch_gemv_mb<T, 1>(A, W, M, Mdev, N, K, e, s);
  else if (M <= 2) launch_gemv_mb<T, 2>(A, W, M, Mdev, N, K, e, s);
  else if (M <= 4) launch_gemv_mb<T, 4>(A, W, M, Mdev, N, K, e, s);
  else launch_gemv_mb<T, 8>(A, W, M, Mdev, N, K, e, s);
}

// register ring depth of the K-split kernel: 4 chunks for the 32 x 16 and
// 32 x 32 tiles (the draft's weight streams: few columns per wave), else 3
template <int MB, int NB, bool PK = false, int NS = (MB == 2 && NB <= 2) ? 4 : 3>
static void launch_ks(const void* A, const void* W, int Mcap, const int* Mdev, int N, int K, int S, const Epi& e,
                      hipStream_t s) {
  const int ntiles = N / (16 * NB), mtiles = (Mcap + 16 * MB - 1) / (16 * MB);
  const int nwg = (ntiles + 7) / 8 * 8 * S * mtiles;
  const int mfast = Mdev == nullptr ? 1 : 0;
  FC_EPI_SWITCH(e.mode, hipLaunchKernelGGL((k_gemm_ks<MB, NB, NS, E, PK>), dim3(nwg), dim3(256), 0, s,
                                           (const bf16_t*)A, (const bf16_t*)W, Mcap, Mdev, N, K, ntiles, S, mtiles,
                                           mfast, e));
}

#define FC_GEMM_LA_NS 3
template <int MB, int NBW>
static void launch_la(const void* A, const void* W, int Mcap, const int* Mdev, int N, int K, int S, const Epi& e,
                      hipStream_t s) {
  const int ntiles = N / (64 * NBW), mtiles = (Mcap + 16 * MB - 1) / (16 * MB);
  const int nwg = (ntiles + 7) / 8 * 8 * S * mtiles;
  const int mfast = Mdev == nullptr ? 1 : 0;
  FC_EPI_SWITCH(e.mode, hipLaunchKernelGGL((k_gemm_la<MB, NBW, FC_GEMM_LA_NS, E>), dim3(nwg), dim3(256), 0, s,
                                           (const bf16_t*)A, (const bf16_t*)W, Mcap, Mdev, N, K, ntiles, S, mtiles,
                                           mfast, e));
}

template <int MB, int NBW>
static void launch_dma(const void* A, const void* W, int Mcap, const int* Mdev, int N, int K, const Epi& e,
                       hipStream_t s) {
  const int ntiles = N / (64 * NBW), mtiles = (Mcap + 16 * MB - 1) / (16 * MB);
  const int nwg = (ntiles + 7) / 8 * 8 * mtiles;
  const int mfast = Mdev == nullptr ? 1 : 0;
  FC_EPI_SWITCH(e.mode, hipLaunchKernelGGL((k_gemm_dma<MB, NBW, E>), dim3(nwg), dim3(256), 0, s, (const bf16_t*)A,
                                           (const bf16_t*)W, Mcap, Mdev, N, K, ntiles, mtiles, mfast, e));
}

// the ring tiles: 64 x 96 with 5 stages (verify c_fc and MLP c_proj), 32 x 32
// with 4 (verify attention c_proj); 2 x 2 waves
template <int MB, int NB, int NSTG, int WM>
static void launch_ring(const void* A, const void* W, int Mcap, const int* Mdev, int N, int K, int S, const Epi& e,
                        hipStream_t s) {
  const int ntiles = N / (16 * NB), mtiles = (Mcap + 16 * MB - 1) / (16 * MB);
  const int nwg = (ntiles + 7) / 8 * 8 * S * mtiles;
  FC_EPI_SWITCH(e.mode, hipLaunchKernelGGL((k_gemm_ring<MB, NB, NSTG, WM, E>), dim3(nwg), dim3(256), 0, s,
                                           (const bf16_t*)A, (const bf16_t*)W, Mcap, Mdev, N, K, ntiles, S, e));
}

template <int EPI, int NB>
static void launch_big_e(const void* A, const void* W, int Mcap, const int* Mdev, int N, int K, int S, const Epi& e,
                         hipStream_t s) {
  const int ntiles = N / (64 * NB), mtiles = (Mcap + 255) / 256;
  const int per_xcd = S == 8 ? ntiles * mtiles : (ntiles * mtiles + 7) / 8;
  hipLaunchKernelGGL((k_gemm_big<EPI, NB>), dim3(8 * per_xcd), dim3(256), 0, s, (const bf16_t*)A, (const bf16_t*)W,
                     Mcap, Mdev, N, K, ntiles, mtiles, per_xcd, S, e);
}
// 256-column tiles unless they leave CUs idle in a single partial wave of
// workgroups and 192 divides N (n_embd-wide outputs: 1536 = 8 x 192)
static int big_tile_blocks(int Mcap, int N) {
  const int mtiles = (Mcap + 255) / 256;
  if (N % 256 == 0 && (N / 256) * mtiles >= 240) return 4;
  return N % 192 == 0 ? 3 : 4;
}
// nb: 32-column blocks per wave (3 or 4), 0 = by big_tile_blocks; S > 1 only with EPI_PARTIAL
static void launch_big(const void* A, const void* W, int Mcap, const int* Mdev, int N, int K, int nb, int S,
                       const Epi& e, hipStream_t s) {
  const bool w192 = e.mode != EPI_QKV && (nb ? nb == 3 : big_tile_blocks(Mcap, N) == 3);
#define BIG_NB(E) (w192 ? launch_big_e<E, 3>(A, W, Mcap, Mdev, N, K, S, e, s) : launch_big_e<E, 4>(A, W, Mcap, Mdev, N, K, S, e, s))
  switch (e.mode) {
    case EPI_STORE: BIG_NB(EPI_STORE); break;
    case EPI_ADD: BIG_NB(EPI_ADD); break;
    case EPI_RELU2: BIG_NB(EPI_RELU2); break;
    case EPI_MLPOUT: BIG_NB(EPI_MLPOUT); break;
    case EPI_PARTIAL: BIG_NB(EPI_PARTIAL); break;
    case EPI_QKV: launch_big_e<EPI_QKV, 4>(A, W, Mcap, Mdev, N, K, 1, e, s); break;
    default: BIG_NB(EPI_SOFTCAP); break;
  }
#undef BIG_NB
}

template <int MB>
static void launch_la_qkv(const void* A, const void* W, int Mcap, const int* Mdev, int N, int K, const Epi& e,
                          hipStream_t s) {
  const int ntiles = N / 128, mtiles = (Mcap + 16 * MB - 1) / (16 * MB);
  const int nwg = (ntiles + 7) / 8 * 8 * mtiles;
  hipLaunchKernelGGL((k_gemm_la<MB, 2, FC_GEMM_LA_NS, EPI_QKV>), dim3(nwg), dim3(256), 0, s, (const bf16_t*)A,
                     (const bf16_t*)W, Mcap, Mdev, N, K, ntiles, 1, mtiles, Mdev == nullptr ? 1 : 0, e);
}

// One plan drives the workspace sizing and the launch. The tile shape and
// the K split are chosen for the typical row count Mtyp (the grid covers
// Mcap rows; tiles past the device-side count exit at once).
struct GemmPlan {
  bool gemv, la, dma, big;  // VALU GEMV (fp32) / LDS-shared-A / LDS-ring / 256 x 256 (else the K-split kernel)
  bool ring;                // deep direct-load ring, 64 x 96 tiles (k_gemm_ring)
  int mb, nb, S;       // k_gemm_ks: 16 mb x 16 nb tile; k_gemm_la, k_gemm_dma: 16 mb x 64 nb tile
};
#ifndef FC_GEMM_DMA
#define FC_GEMM_DMA 1
#endif
#ifndef FC_GEMM_RING
#define FC_GEMM_RING 1
#endif
// The ring tiles for the verify c_fc (64 x 96, ReLU^2 with the folded
// RMSNorm) and the folded-norm attention c_proj (32 x 32): correct (the GPU
// suite passes with them) but not faster in the cfg4 round (alternating
// builds, three runs each: c_fc 4.868-4.881 vs 4.837-4.840 ms, attention
// c_proj 4.833-4.838 ms), so both stay on k_gemm_dma / k_gemm_ks.
#ifndef FC_RING_FC
#define FC_RING_FC 0
#endif
#ifndef FC_RING_APROJ
#define FC_RING_APROJ 0
#endif
// Row counts from which the layer GEMMs below the 256 x 256 kernel take the
// larger tiles (large-batch verify chunks, e.g. 128 rows x 9 tokens): c_fc
// on the LDS-shared 128 x 128 tile, QKV with its fused prologue on 64 x 128,
// the MLP c_proj unsplit on the LDS-ring 64 x 64 tile, the folded-norm
// attention c_proj on 32 x 64. A sweep of the
// three shapes at 224 / 448 / 672 / 896 / 1152 rows put the crossover
// between 672 and 896 rows.
#ifndef FC_MID_M
#define FC_MID_M 832
#endif
// residual-stream GEMMs of verify chunks from FC_MID_M rows on the 256-row
// tiles with a K split (MFMA-bound there: 1280 x 1536 x 6144 is 24 GFLOP)
#ifndef FC_BIG_SPLIT
#define FC_BIG_SPLIT 1
#endif
// column blocks of 64 per tile of the draft lm_head (up to 32 rows): with the
// vocab pass in its epilogue, 32 x 128 tiles (2) measured 4.780-4.788 vs
// 4.773-4.775 ms per cfg4 round (alternating builds)
#ifndef FC_DRAFT_HEAD_NB
#define FC_DRAFT_HEAD_NB 1
#endif
// Tile shape and K split by typical row count, from sweeps on MI355X at the
// engine's shapes (N = 1536 / 4608 / 6144 / 65536, K = 1536 / 6144).
static GemmPlan plan_gemm(int Mtyp, int N, int K, int dtype, bool can_split) {
  GemmPlan p{};
  p.S = 1;
  if (dtype == FC_F32) {
    p.gemv = true;
    return p;
  }
  if (Mtyp >= (N >= 16384 ? FC_BIG_HEAD_M : FC_BIG_M) && N % 256 == 0 && K % 128 == 0) {
    // prefill chunks: 256 x 256 (or 256 x 192) tiles, MFMA-bound, when there
    // are enough of them to occupy the CUs (verify-size M of ~1200 rows gives
    // 5 M tiles: the 64-row kernels are faster there)
    const int mt = (Mtyp + 255) / 256;
    const int tiles = std::max(mt * (N / 256), N % 192 == 0 ? mt * (N / 192) : 0);
    if (tiles >= FC_BIG_MIN_TILES) {
      p.big = true;
      return p;
    }
  }
  if (can_split && FC_BIG_SPLIT && Mtyp >= FC_MID_M && K % 1024 == 0) {
    // large verify chunks (cfg5: 1152-1280 rows), residual-stream GEMMs with
    // a deep K (the MLP c_proj): 256-row tiles with the K range split 8
    // ways, one split per XCD, when a split's 24-32 output tiles fill that
    // XCD's 32 CUs once; the next RMSNorm sums the partials
    const int mt = (Mtyp + 255) / 256;
    for (int nb = 4; nb >= 3; --nb) {
      const int tiles = N % (64 * nb) == 0 ? mt * (N / (64 * nb)) : 0;
      if (tiles >= 24 && tiles <= 32) {
        p.big = true;
        p.nb = nb;
        p.S = 8;
        return p;
      }
    }
  }
  const int C = K / 64;
  const int s_max = std::max(1, std::min(C / 4, FC_MAX_SPLIT));  // >= 1 chunk per wave
  if (Mtyp <= 16) {
    // one 16-row tile: fill the GPU with column tiles and K splits
    p.mb = 1;
    p.nb = 4;
    const int wgs = std::max(1, N / 64);
    if (can_split && wgs < 256) p.S = std::min((256 + wgs - 1) / wgs, s_max);
  } else if (Mtyp <= 32) {
    if (!can_split && N >= 16384 && N % (64 * FC_DRAFT_HEAD_NB) == 0) {  // draft lm_head: LDS-shared rows
      p.la = true;
      p.mb = 2;
      p.nb = FC_DRAFT_HEAD_NB;  // 64-column tiles (or 128)
      return p;
    }
    p.mb = 2;
    p.nb = 2;
    if (can_split) {  // n_embd columns: 16-column tiles and a K split fill the GPU
      p.nb = 1;
      p.S = std::min(K > 2048 ? 8 : 3, s_max);
    }
  } else if (can_split) {
    if (Mtyp >= FC_MID_M && N % 64 == 0 && FC_GEMM_DMA) {  // enough 64 x 64 tiles: no K split
      p.dma = true;
      p.mb = 4;
      p.nb = 1;
      return p;
    }
    // verify chunks below FC_MID_M rows whose residual GEMM has n_embd = a
    // multiple of 96 columns: the deep-ring 64 x 96 tiles with a 4-way split
    // (cfg4's MLP c_proj: 16 x 4 tiles x 4 splits = 256 workgroups)
    if (FC_GEMM_RING && Mtyp > 160 && N % 96 == 0 && C % 4 == 0 && s_max >= 4) {
      p.ring = true;
      p.mb = 4;
      p.nb = 6;
      p.S = 4;
      return p;
    }
    // 33-160 rows (large-batch draft steps): 32 x 32 tiles, 4-way split;
    // from there (verify chunks) 32 x 64, 3-way
    p.mb = 2;
    p.nb = Mtyp <= 160 ? 2 : 4;
    p.S = std::min(Mtyp <= 160 ? 4 : 3, s_max);
  } else if (Mtyp >= 128 && N % 128 == 0) {
    // verify / prefill rows: a wide output (lm_head) takes the LDS-shared
    // kernel's 128 x 128 tiles; the layer GEMMs the LDS-ring kernel's 64 x 64
    // (the fused QKV epilogue takes its 32 x 128: one head per tile)
    if (N >= 16384 || !FC_GEMM_DMA) {
      p.la = true;
      p.mb = N >= 16384 ? 8 : 2;
      p.nb = 2;
    } else {
      p.dma = true;
      p.mb = 4;
      p.nb = 1;
    }
    return p;
  } else {
    p.mb = 2;
    p.nb = 4;
  }
  while (p.nb > 1 && N % (16 * p.nb) != 0) p.nb /= 2;
  if (p.nb == 1 && p.mb != 2) p.nb = 2;  // instantiated shapes: (1,2|4), (2,1|2|4)
  return p;
}

// c_fc (the ReLU^2 epilogue): verify rows (161 .. FC_MID_M - 1) on the ring's
// 64 x 96 tiles; from FC_MID_M rows the LDS-shared 128 x 128 tile
static GemmPlan plan_relu2(int Mtyp, int N, int K, int dtype) {
  GemmPlan p = plan_gemm(Mtyp, N, K, dtype, false);
  if (FC_GEMM_RING && FC_RING_FC && dtype == FC_BF16 && !p.big && Mtyp > 160 && Mtyp < FC_MID_M && N % 96 == 0) {
    p = GemmPlan{};
    p.S = 1;
    p.ring = true;
    p.mb = 4;
    p.nb = 6;
    return p;
  }
  if (dtype == FC_BF16 && !p.big && Mtyp >= FC_MID_M && N % 128 == 0) {
    p = GemmPlan{};
    p.S = 1;
    p.la = true;
    p.mb = 8;
    p.nb = 2;
  }
  return p;
}

// Up to this many typical rows (one-row decode: cfg2's 5-token verify and
// 1-token draft steps) the QKV GEMM takes one-head 32 x 128 tiles and
// finishes the attention prologue itself, saving the k_prologue dispatch:
// cfg2 0.923-0.927 vs 0.952-0.956 ms per round (alternating builds). At 32
// rows (cfg4's draft steps: 36 workgroups over 14 MB) the separate
// prologue is faster.
#ifndef FC_QKV_TINY_M
#define FC_QKV_TINY_M 16
#endif
bool fc_gemm_fuses_qkv(int Mtyp, int N, int K, int dtype, int head_dim) {
  if (dtype != FC_BF16 || head_dim != 128 || N % 128 != 0 || K % 64 != 0) return false;
  if (Mtyp <= FC_QKV_TINY_M) return true;
  const GemmPlan p = plan_gemm(Mtyp, N, K, dtype, false);
  // the QKV tile itself is k_gemm_la's 32 x 128 (64 x 128 from FC_MID_M rows), or a 128 x 128 quadrant of k_gemm_big
  return p.big || p.dma || (p.la && p.mb == 2 && p.nb == 2);
}

// The EPI_ADD GEMM that writes the bf16 copy of x (attention c_proj, bf16):
// unsplit K-split kernel, 32 x 16 tiles for draft rows, 32 x 32 for verify rows.
static GemmPlan plan_fold_add(int Mtyp, int N) {
  GemmPlan p{};
  p.S = 1;
  if (FC_GEMM_RING && FC_RING_APROJ && Mtyp > 160 && Mtyp < FC_MID_M && N % 32 == 0) {  // verify rows: the ring's 32 x 32 tiles
    p.ring = true;
    p.mb = 2;
    p.nb = 2;
    return p;
  }
  p.mb = Mtyp <= 16 ? 1 : 2;
  p.nb = Mtyp <= 16 ? 2 : (Mtyp <= 32 ? 1 : (Mtyp < FC_MID_M ? 2 : 4));
  while (p.nb > 1 && N % (16 * p.nb) != 0) p.nb /= 2;
  if (p.nb == 1 && p.mb != 2) p.nb = 2;
  return p;
}
int fc_gemm_fold_tiles(int Mtyp, int N) { return N / (16 * plan_fold_add(Mtyp, N).nb); }
// the consumer (c_fc: N = 4 D, K = D) prefetches FC_RMS_REG tiles per thread
// with 256 / MT threads per row
bool fc_gemm_fold_ok(int Mtyp, int D) {
  const GemmPlan c = plan_relu2(Mtyp, 4 * D, D, FC_BF16);
  return !c.gemv && !c.big && fc_gemm_fold_tiles(Mtyp, D) <= FC_RMS_REG * (256 / (16 * c.mb));
}

int64_t fc_gemm_part_bytes(int Mtyp, int Mcap, int N, int K, int dtype) {
  if (Mtyp <= 0 || Mcap <= 0 || N <= 0 || K <= 0) return 0;
  GemmPlan p = plan_gemm(Mtyp, N, K, dtype, true);  // fp32 GEMMs never split
  return p.S > 1 ? fc_align((int64_t)p.S * Mcap * N * 4) : 0;
}

int fc_launch_gemm(const void* A, const void* W, int Mcap, const int* Mdev, int Mtyp, int N, int K, int dtype,
                   const Epi& e, const GemmWork& gw, hipStream_t s, int* splits) {
  if (splits) *splits = 1;
  if (Mcap <= 0 || N <= 0) return FC_OK;
  FC_CHECK_ARG(K > 0 && K % 8 == 0, "gemm K must be a positive multiple of 8");
  if (Mtyp <= 0 || Mtyp > Mcap) Mtyp = Mcap;
  FC_CHECK_ARG(dtype == FC_F32 || (K % 64 == 0 && N % 32 == 0),
               "bf16 GEMM needs K % 64 == 0 and N % 32 == 0 (fragment-order operands)");
  if (e.mode == EPI_QKV) {
    FC_CHECK_ARG(fc_gemm_fuses_qkv(Mtyp, N, K, dtype, 128), "EPI_QKV needs the 32 x 128 bf16 tile");
    if (plan_gemm(Mtyp, N, K, dtype, false).big) launch_big(A, W, Mcap, Mdev, N, K, 0, 1, e, s);
    else if (Mtyp >= FC_MID_M) launch_la_qkv<4>(A, W, Mcap, Mdev, N, K, e, s);  // 64 x 128 tiles
    else launch_la_qkv<2>(A, W, Mcap, Mdev, N, K, e, s);
    FC_LAUNCH_CHECK();
    return FC_OK;
  }
  const bool can_split = splits != nullptr && gw.part != nullptr;
  GemmPlan p = e.mode == EPI_RELU2 && !can_split ? plan_relu2(Mtyp, N, K, dtype) : plan_gemm(Mtyp, N, K, dtype, can_split);
  if (e.mode == EPI_ADD && e.xa != nullptr) {
    FC_CHECK_ARG(dtype == FC_BF16 && e.ssq != nullptr && !can_split, "folded-norm GEMM: bf16, ssq, no split");
    p = plan_fold_add(Mtyp, N);
  }
  if (p.S > 1 && (int64_t)p.S * Mcap * N * 4 > gw.part_bytes) p.S = 1;
  FC_CHECK_ARG(e.vp == nullptr || (e.mode == EPI_SOFTCAP && p.la && p.S == 1 && p.mb % 2 == 0 &&
                                   e.vp_ld == N / (64 * (p.mb == 8 || p.nb != 1 ? 2 : 1))),
               "vocab-pass partials: an unsplit EPI_SOFTCAP GEMM on the LDS-shared kernel, vp_ld = its column tiles");
  Epi ee = e;
  if (p.S > 1) {
    ee.mode = EPI_PARTIAL;
    ee.part = gw.part;
    ee.part_rows = Mcap;
    ee.ldo = N;
    *splits = p.S;
  }
  if (p.gemv) {
    launch_gemv<float>(A, W, Mcap, Mdev, N, K, ee, s);
  } else if (p.big) {
    FC_CHECK_ARG(ee.rms_in == nullptr && ee.xa == nullptr, "the 256 x 256 GEMM has no folded-norm epilogue");
    FC_CHECK_ARG(p.S == 1 || (p.S == 8 && ee.mode == EPI_PARTIAL && K % 1024 == 0),
                 "the 256 x 256 GEMM splits K only 8 ways, in multiples of 4 k steps per split");
    launch_big(A, W, Mcap, Mdev, N, K, p.nb, p.S, ee, s);
  } else if (p.ring) {
    if (p.mb == 2) launch_ring<2, 2, 4, 2>(A, W, Mcap, Mdev, N, K, p.S, ee, s);  // 32 x 32, 4 stages
    else launch_ring<4, 6, 5, 2>(A, W, Mcap, Mdev, N, K, p.S, ee, s);           // 64 x 96, 5 stages
  } else if (p.dma) {
    launch_dma<4, 1>(A, W, Mcap, Mdev, N, K, ee, s);
  } else if (p.la) {
    if (p.mb == 8) launch_la<8, 2>(A, W, Mcap, Mdev, N, K, p.S, ee, s);
    else if (p.nb == 1) launch_la<2, 1>(A, W, Mcap, Mdev, N, K, p.S, ee, s);
    else launch_la<2, 2>(A, W, Mcap, Mdev, N, K, p.S, ee, s);
  } else if (p.mb == 1) {
    if (p.nb == 4) launch_ks<1, 4, true>(A, W, Mcap, Mdev, N, K, p.S, ee, s);
    else launch_ks<1, 2, true>(A, W, Mcap, Mdev, N, K, p.S, ee, s);
  } else {
    if (p.nb == 4) launch_ks<2, 4, true>(A, W, Mcap, Mdev, N, K, p.S, ee, s);
    else if (p.nb == 2) launch_ks<2, 2, true>(A, W, Mcap, Mdev, N, K, p.S, ee, s);
    else launch_ks<2, 1, true>(A, W, Mcap, Mdev, N, K, p.S, ee, s);
  }
  FC_LAUNCH_CHECK();
  return FC_OK;
}

int fc_gemm_vocab_tiles(int M, int N, int K, int dtype) {
  if (M <= 0 || N <= 0 || dtype != FC_BF16 || K % 64 != 0 || N % 32 != 0) return 0;
  const GemmPlan p = plan_gemm(M, N, K, dtype, false);
  if (!p.la || p.S != 1 || p.mb % 2 != 0) return 0;
  return N / (64 * (p.mb == 8 || p.nb != 1 ? 2 : 1));  // launch_la<8, 2>, <2, 1> or <2, 2>
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
  return fc_launch_gemm(A, W, M, nullptr, M, N, K, dtype, e, GemmWork{}, (hipStream_t)stream, nullptr);
}

// Fragment-order copy of a row-major bf16 matrix src[rows][K] into
// dst[round16(rows)][K] (padding rows zero); one thread per 16-byte group.
__global__ __launch_bounds__(256) void k_pack_frag(const bf16_t* __restrict__ src, bf16_t* __restrict__ dst,
                                                   int rows, int K) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t groups = round16(rows) * (K / 8);
  if (t >= groups) return;
  const int64_t blk = t >> 6;  // 64 groups per 16 x 32 block
  const int lane = (int)(t & 63);
  const int KS = K >> 5;
  const int64_t rb = blk / KS;
  const int ks = (int)(blk - rb * KS);
  const int64_t r = rb * 16 + (lane & 15);
  const int k = ks * 32 + (lane >> 4) * 8;
  uint4 v = {0u, 0u, 0u, 0u};
  if (r < rows) v = *(const uint4*)(src + r * K + k);
  *(uint4*)(dst + t * 8) = v;
}

extern "C" int32_t fc_pack_operand(const void* src, void* dst, int32_t rows, int32_t K, void* stream) {
  FC_CHECK_ARG(src && dst && src != dst, "pointers (distinct, non-null)");
  FC_CHECK_ARG(rows > 0 && K > 0 && K % 32 == 0, "rows > 0 and K % 32 == 0");
  const int64_t groups = round16(rows) * (K / 8);
  hipLaunchKernelGGL(k_pack_frag, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const bf16_t*)src, (bf16_t*)dst, rows, K);
  FC_LAUNCH_CHECK();
  return FC_OK;
}
