// Top-k selection over chunked candidates and the order-preserving float
// keys it uses, shared by the sampling kernels and the embedding kernel that
// finishes a top-k draft step for the next one (fc_vocab.h draft_merge_row).
#pragma once
#include "fc_common.h"
#include "fc_internal.h"

// order-preserving uint32 key of a float, and back
__device__ __forceinline__ uint32_t mono(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float unmono(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
__device__ __forceinline__ bool kept(float z, int idx, uint32_t tau_key, int tie_idx) {
  const uint32_t k = mono(z);
  return k > tau_key || (k == tau_key && idx <= tie_idx);
}

// ---------------------------------------------------------------------------
// Top-k rows split over many workgroups (0 < top_k <= TK_MAX, T > 0): every
// 1024-entry chunk of a row keeps its own top-k candidates (larger value
// first, lower index first among equal values), the row's keep set being a
// subset of their union (an entry with top_k entries ahead of it in its own
// chunk has them ahead of it in the row); then one workgroup per row selects
// the keep set among the candidates and computes the statistics. For a draw (Gumbel-max over
// log(max(p, 1e-10)) + G, flaxchat/engine.py:478-482) the candidates are
// scored with their own noise; every other entry has p = 0, so a chunk only
// reports the largest G among its non-candidates.
// ---------------------------------------------------------------------------
#define TK_EPL 16                 // entries per lane of the chunk pass
#define TK_CH (64 * TK_EPL)       // entries per chunk (one wave)
#define TK_MAX 64                 // candidates per chunk: top_k <= TK_MAX
#define TK_NCH 64                 // chunks per row: V <= TK_NCH * TK_CH
#define TK_THR 256
#define TK_SPT (TK_NCH * TK_MAX / TK_THR)  // candidate slots per thread of the per-row pass
struct TkChunk {      // one chunk of one row
  float g; int gi;    // largest G among the chunk's non-candidates (draw only) and its index
  int n;              // candidates kept (min(top_k, entries in the chunk))
  uint32_t kmax;      // order-preserving key of the chunk's largest entry
  float z[TK_MAX];    // candidates in index order, their indices and (draw) their G
  int idx[TK_MAX];
  float gz[TK_MAX];
};

// Counts over the wave from ballots (a compare mask and a population
// count, no cross-lane data movement); every lane of the wave takes part.
// lanes whose `pred` holds (uniform over the wave)
__device__ __forceinline__ int wave_count(bool pred) { return __popcll(__ballot(pred)); }
// lanes below this one whose `pred` holds
__device__ __forceinline__ int lanes_below(bool pred) {
  const uint64_t m = __ballot(pred);
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}
// exclusive prefix sum over the wave's lanes of v in [0, 2^BITS)
template <int BITS>
__device__ __forceinline__ int wave_excl_small(int v) {
  int r = 0;
#pragma unroll
  for (int b = 0; b < BITS; ++b) r += lanes_below((v >> b) & 1) << b;
  return r;
}
// sum over the wave's lanes of v in [0, 2^BITS) (uniform)
template <int BITS>
__device__ __forceinline__ int wave_sum_small(int v) {
  int r = 0;
#pragma unroll
  for (int b = 0; b < BITS; ++b) r += wave_count((v >> b) & 1) << b;
  return r;
}

// The kk-th largest order-preserving key among a wave's entries (N per lane,
// `ok` marks real ones), known to lie in [lo, hi]: the largest t with
// #{key >= t} >= kk, by binary search counted with ballots; also #{key > t}.
// lo and hi are uniform over the wave, and so is the result.
template <int N>
__device__ __forceinline__ uint32_t wave_kth_key(const uint32_t (&key)[N], const bool (&ok)[N], int kk, uint32_t lo,
                                                 uint32_t hi, int& ngt) {
  while (lo < hi) {
    const uint32_t mid = lo + (uint32_t)(((uint64_t)hi - lo + 1) >> 1);
    int n = 0;
#pragma unroll
    for (int q = 0; q < N; ++q) n += wave_count(ok[q] && key[q] >= mid);
    if (n >= kk) lo = mid;
    else hi = mid - 1u;
  }
  int g = 0;
#pragma unroll
  for (int q = 0; q < N; ++q) g += wave_count(ok[q] && key[q] > lo);
  ngt = g;
  return lo;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, WAVE));
  return v;
}
// Entries the search keeps after the lower bound: at most this many go
// through the narrow search (2 per lane of the chunk pass, 4 per lane of the
// row pass), more take the search over every entry.
#define TK_NARROW_WAVE 128
#define TK_NARROW_ROW 256

// Keep flags of a wave's entries (index order = (lane, q) order) for the
// threshold key tau: every entry above it and the first need equal to it;
// *last_eq = the index of the need-th equal entry (written by its lane).
template <int N>
__device__ __forceinline__ void wave_keep(const uint32_t (&key)[N], const bool (&ok)[N], const int (&idx)[N],
                                          uint32_t tau, int need, bool (&in)[N], int* last_eq) {
  int neq = 0;
#pragma unroll
  for (int q = 0; q < N; ++q) neq += ok[q] && key[q] == tau;
  static_assert(N < 32, "per-lane counts below 2^5");
  int eq_before = wave_excl_small<5>(neq);
#pragma unroll
  for (int q = 0; q < N; ++q) {
    in[q] = false;
    if (ok[q]) {
      const uint32_t k = key[q];
      if (k > tau) {
        in[q] = true;
      } else if (k == tau) {
        ++eq_before;
        in[q] = eq_before <= need;
        if (last_eq != nullptr && eq_before == need) *last_eq = idx[q];
      }
    }
  }
}

// Keep set and statistics of one logits row from its chunks' candidates, by
// one workgroup (row_stats_block's result; tie_idx is the last kept index
// equal to tau): the binary search over the candidate keys counted over the
// block; with `draw`, the Gumbel-max token from the candidates' stored G and
// the chunks' largest G outside them (p = 0 there: log(1e-10) + G).
struct TkRow {
  fc_rowstat st;
  int tok;
};
__device__ __forceinline__ TkRow tk_finish_row(const TkChunk* __restrict__ ch, int nch, int V, int top_k, float T,
                                               bool draw) {
  __shared__ int red[2][TK_THR / 64];
  __shared__ int tie_sm;
  __shared__ float redv[16];
  __shared__ int redi[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // slot q of thread t: candidate j of chunk cc for t TK_SPT + q = cc TK_MAX + j (index order);
  // a thread's TK_SPT slots are consecutive candidates of one chunk, loaded
  // as whole 16-byte groups together with the chunk's count (one round trip;
  // slots past the count are masked afterwards)
  static_assert(TK_MAX % TK_SPT == 0 && TK_SPT % 4 == 0, "a thread's slots: 16-byte groups of one chunk");
  float zv[TK_SPT], gv[TK_SPT];
  int iv[TK_SPT];
  bool ok[TK_SPT];
  {
    const int cc = threadIdx.x * TK_SPT / TK_MAX, j0 = threadIdx.x * TK_SPT - cc * TK_MAX;
    const TkChunk* c = ch + min(cc, nch - 1);
    const int n = c->n;
    float4 z4[TK_SPT / 4], g4[TK_SPT / 4];
    int4 i4[TK_SPT / 4];
#pragma unroll
    for (int u = 0; u < TK_SPT / 4; ++u) {
      z4[u] = *(const float4*)&c->z[j0 + 4 * u];
      i4[u] = *(const int4*)&c->idx[j0 + 4 * u];
      g4[u] = draw ? *(const float4*)&c->gz[j0 + 4 * u] : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int q = 0; q < TK_SPT; ++q) {
      const float4 zz = z4[q >> 2], gg = g4[q >> 2];
      const int4 ii = i4[q >> 2];
      const int w = q & 3;
      ok[q] = cc < nch && j0 + q < n;
      zv[q] = ok[q] ? (w == 0 ? zz.x : w == 1 ? zz.y : w == 2 ? zz.z : zz.w) : -INFINITY;
      iv[q] = ok[q] ? (w == 0 ? ii.x : w == 1 ? ii.y : w == 2 ? ii.z : ii.w) : 0x7fffffff;
      gv[q] = ok[q] && draw ? (w == 0 ? gg.x : w == 1 ? gg.y : w == 2 ? gg.z : gg.w) : 0.f;
    }
  }
  const int kk = min(top_k, V);
  uint32_t kz[TK_SPT];
#pragma unroll
  for (int q = 0; q < TK_SPT; ++q) kz[q] = mono(zv[q]);
  // lower bound for the row's kk-th largest key: the kk-th largest of the
  // chunks' maxima (kk entries reach it), and the row's largest key
  __shared__ uint32_t bound_sm[2], tau_sm;
  __shared__ int cnt_sm[TK_THR / 64];
  __shared__ uint32_t cs[TK_NARROW_ROW];
  static_assert(TK_NCH <= 64, "one chunk maximum per lane of a wave");
  if (wave == 0) {
    const TkChunk* cl = ch + min(lane, nch - 1);  // count and maximum loaded together
    const int cn = cl->n;
    const uint32_t ckmax = cl->kmax;
    const bool has = lane < nch && cn > 0;
    const uint32_t cm[1] = {has ? ckmax : 0u};
    const bool co[1] = {has};
    const uint32_t rmax = wave_max_u32(cm[0]);
    uint32_t tlo = 0u;
    if (wave_count(has) >= kk) {
      int unused;
      tlo = wave_kth_key<1>(cm, co, kk, 0u, rmax, unused);
    }
    if (lane == 0) {
      bound_sm[0] = tlo;
      bound_sm[1] = rmax;
    }
  }
  __syncthreads();
  const uint32_t tlo = bound_sm[0], rmax = bound_sm[1];
  int cnt = 0;
#pragma unroll
  for (int q = 0; q < TK_SPT; ++q) cnt += ok[q] && kz[q] >= tlo;
  static_assert(TK_SPT < 32, "per-thread counts below 2^5");
  const int wcnt = wave_sum_small<5>(cnt);
  if (lane == 0) cnt_sm[wave] = wcnt;
  __syncthreads();
  int total = 0, before = 0;
#pragma unroll
  for (int w = 0; w < TK_THR / 64; ++w) {
    total += cnt_sm[w];
    if (w < wave) before += cnt_sm[w];
  }
  uint32_t tau;
  if (total <= TK_NARROW_ROW) {
    // the few keys at or above the bound, searched by one wave
    int p = before + wave_excl_small<5>(cnt);
#pragma unroll
    for (int q = 0; q < TK_SPT; ++q)
      if (ok[q] && kz[q] >= tlo) cs[p++] = kz[q];
    __syncthreads();
    if (wave == 0) {
      uint32_t k4[4];
      bool o4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        o4[u] = lane + 64 * u < total;
        k4[u] = o4[u] ? cs[lane + 64 * u] : 0u;
      }
      int unused;
      const uint32_t t = wave_kth_key<4>(k4, o4, kk, tlo, rmax, unused);
      if (lane == 0) tau_sm = t;
    }
    __syncthreads();
    tau = tau_sm;
  } else {
    uint32_t lo = 0u, hi = rmax;
    int it = 0;
    while (lo < hi) {  // the same sequence in every thread
      const uint32_t mid = lo + (uint32_t)(((uint64_t)hi - lo + 1) >> 1);
      int n = 0;
#pragma unroll
      for (int q = 0; q < TK_SPT; ++q) n += wave_count(ok[q] && kz[q] >= mid);
      if (lane == 0) red[it & 1][wave] = n;  // alternating buffers: one barrier per step
      __syncthreads();
      int tot = 0;
#pragma unroll
      for (int w = 0; w < TK_THR / 64; ++w) tot += red[it & 1][w];
      if (tot >= kk) lo = mid;
      else hi = mid - 1u;
      ++it;
    }
    tau = lo;
  }
  int ngt = 0, neq = 0;
#pragma unroll
  for (int q = 0; q < TK_SPT; ++q) {
    ngt += ok[q] && mono(zv[q]) > tau;
    neq += ok[q] && mono(zv[q]) == tau;
  }
  static_assert(TK_SPT < 32, "per-thread counts below 2^5");
  const int wgt = wave_sum_small<5>(ngt), weq_ex = wave_excl_small<5>(neq), weq = wave_sum_small<5>(neq);
  __syncthreads();
  if (lane == 0) {
    red[0][wave] = wgt;
    red[1][wave] = weq;
  }
  __syncthreads();
  int gt = 0, eq_before = weq_ex;
#pragma unroll
  for (int w = 0; w < TK_THR / 64; ++w) {
    gt += red[0][w];
    if (w < wave) eq_before += red[1][w];
  }
  const int need = kk - gt;
  bool in[TK_SPT];
#pragma unroll
  for (int q = 0; q < TK_SPT; ++q) {
    in[q] = false;
    if (ok[q]) {
      const uint32_t k = mono(zv[q]);
      if (k > tau) {
        in[q] = true;
      } else if (k == tau) {
        ++eq_before;
        in[q] = eq_before <= need;
        if (eq_before == need) tie_sm = iv[q];  // exactly one slot of the block
      }
    }
  }
  __syncthreads();
  const int tie_idx = tie_sm;
  float bz = -INFINITY;
  int bzi = 0x7fffffff;
#pragma unroll
  for (int q = 0; q < TK_SPT; ++q)
    if (in[q]) argmax_merge(bz, bzi, zv[q], iv[q]);
  block_argmax(bz, bzi, redv, redi);
  const float mx = bz / T;  // max of z / T over the keep set
  float sum = 0.f;
#pragma unroll
  for (int q = 0; q < TK_SPT; ++q)
    if (in[q]) sum += expf(zv[q] / T - mx);
  sum = block_sum(sum, redv);
  TkRow res;
  res.st = fc_rowstat{};
  res.st.mx = mx;
  res.st.sum = sum;
  res.st.tau = unmono(tau);
  res.st.tie_idx = tie_idx;
  res.st.argmax = bzi;
  res.tok = bzi;
  if (draw) {
    const float lfl = logf(1e-10f);
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int q = 0; q < TK_SPT; ++q)
      if (ok[q]) {
        // outside the keep set p = 0, whose log(max(p, 1e-10)) is lfl
        const float lp = in[q] ? logf(fmaxf(expf(zv[q] / T - mx) / sum, 1e-10f)) : lfl;
        argmax_merge(bv, bi, lp + gv[q], iv[q]);
      }
    for (int cc = threadIdx.x; cc < nch; cc += TK_THR) argmax_merge(bv, bi, lfl + ch[cc].g, ch[cc].gi);
    block_argmax(bv, bi, redv, redi);
    res.tok = bi;
  }
  return res;
}

// Draft step i with a top-k filter: statistics and proposal d_{i+1}, one
// workgroup per row.
