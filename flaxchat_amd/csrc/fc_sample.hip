// Vocab-wide sampling, accept/reject and the device-side round bookkeeping.
//
// Restates flaxchat/engine.py:461-482 (top-k filter, probabilities,
// categorical draw), :525-592 (accept / reject / residual / bonus) and
// replaces the full re-prefill of :593-606 by length-pointer rollback.
//
// Random stream: Philox4x32-10, key = seed, counter = (element / 4, row,
// round, slot); slots: draft sample i -> i, accept uniform i -> 16 + i,
// rejection draw -> 48, bonus draw -> 49 (generate_fast: round = step, slot 0).
// A categorical draw is Gumbel-max over log(max(p, 1e-10)), the same method
// as jax.random.categorical on the reference's log(max(p, 1e-10)) input.
#include "fc_common.h"
#include "fc_internal.h"
#include "fc_topk.h"
#include "fc_vocab.h"
#include <mutex>

#define SLOT_ACCEPT 16
#define SLOT_REJECT 48
#define SLOT_BONUS 49
#define NTHR 1024
#define BIG_POS 0x3fffffff

// ---------------------------------------------------------------------------
// error plumbing, version, graphs
// ---------------------------------------------------------------------------
static thread_local std::string g_err;
void fc_set_error(const std::string& s) { g_err = s; }
extern "C" const char* fc_last_error(void) { return g_err.c_str(); }
extern "C" int32_t fc_version(void) { return 100; }

extern "C" int32_t fc_graph_begin(void* stream) {
  // the allocation-free attention's scratch address is a runtime lookup: done
  // here, before the capture, so captured calls only read the cached address
  const int rc = fc_noalloc_prepare((hipStream_t)stream);
  if (rc != FC_OK) return rc;
  FC_HIP(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal));
  return FC_OK;
}
extern "C" int32_t fc_graph_end(void* stream, void** exec_out) {
  FC_CHECK_ARG(exec_out, "exec_out");
  hipGraph_t g = nullptr;
  FC_HIP(hipStreamEndCapture((hipStream_t)stream, &g));
  hipGraphExec_t ex = nullptr;
  hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  if (e != hipSuccess) {
    fc_set_error(std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    return FC_ERR_HIP;
  }
  *exec_out = (void*)ex;
  return FC_OK;
}
extern "C" int32_t fc_graph_launch(void* exec, void* stream) {
  FC_CHECK_ARG(exec, "exec");
  FC_HIP(hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)stream));
  return FC_OK;
}
extern "C" int32_t fc_graph_destroy(void* exec) {
  if (exec) FC_HIP(hipGraphExecDestroy((hipGraphExec_t)exec));
  return FC_OK;
}

// ---------------------------------------------------------------------------
// Row statistics (block of NTHR threads per row)
// ---------------------------------------------------------------------------

struct StatSmem {
  unsigned hist[256];
  float redv[16];
  int redi[16];
  unsigned cnt[NTHR];
  int sel, remaining, cnt_eq, tie_idx;
  fc_rowstat res;  // the row's statistics, for the block's own use
};

// lax.top_k keep-set (exactly k entries; larger value first, lower index
// first among equal values) by 8-bit radix select over order-preserving
// keys, then max / normaliser of z/T over the kept set and the argmax.
__device__ void row_stats_block(const float* __restrict__ z, int V, float T, int top_k, fc_rowstat* out,
                                StatSmem& sm) {
  const int tid = threadIdx.x;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = tid; i < V; i += NTHR) argmax_merge(bv, bi, z[i], i);
  block_argmax(bv, bi, sm.redv, sm.redi);
  const int amax = bi;
  uint32_t tau_key = mono(-INFINITY);
  int tie_idx = V;
  if (T > 0.f && top_k > 0 && top_k < V) {
    uint32_t prefix = 0, maskbits = 0;
    if (tid == 0) sm.remaining = top_k;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = tid; i < 256; i += NTHR) sm.hist[i] = 0;
      __syncthreads();
      for (int i = tid; i < V; i += NTHR) {
        const uint32_t k = mono(z[i]);
        if ((k & maskbits) == prefix) atomicAdd(&sm.hist[(k >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        unsigned cum = 0;
        int rem = sm.remaining;
        for (int d = 255; d >= 0; --d) {
          const unsigned h = sm.hist[d];
          if (cum + h >= (unsigned)rem) {
            sm.sel = d;
            sm.remaining = rem - (int)cum;
            sm.cnt_eq = (int)h;
            break;
          }
          cum += h;
        }
      }
      __syncthreads();
      prefix |= ((uint32_t)sm.sel) << shift;
      maskbits |= 0xffu << shift;
    }
    tau_key = prefix;
    const int need = sm.remaining, cnt_eq = sm.cnt_eq;
    if (need < cnt_eq) {
      // index of the need-th entry equal to tau, in index order
      const int chunk = (V + NTHR - 1) / NTHR;
      const int lo = tid * chunk, hi = min(V, lo + chunk);
      unsigned c = 0;
      for (int i = lo; i < hi; ++i) c += mono(z[i]) == tau_key;
      sm.cnt[tid] = c;
      __syncthreads();
      if (tid == 0) {
        unsigned acc = 0;
        for (int t = 0; t < NTHR; ++t) {
          const unsigned v = sm.cnt[t];
          sm.cnt[t] = acc;
          acc += v;
        }
      }
      __syncthreads();
      const unsigned before = sm.cnt[tid];
      if (before < (unsigned)need && before + c >= (unsigned)need) {
        unsigned k = before;
        for (int i = lo; i < hi; ++i)
          if (mono(z[i]) == tau_key && ++k == (unsigned)need) {
            sm.tie_idx = i;
            break;
          }
      }
      __syncthreads();
      tie_idx = sm.tie_idx;
    }
  }
  float mx = 0.f, sum = 1.f;
  if (T > 0.f) {
    float m = -INFINITY;
    for (int i = tid; i < V; i += NTHR)
      if (kept(z[i], i, tau_key, tie_idx)) m = fmaxf(m, z[i] / T);
    mx = block_max(m, sm.redv);
    float s = 0.f;
    for (int i = tid; i < V; i += NTHR)
      if (kept(z[i], i, tau_key, tie_idx)) s += expf(z[i] / T - mx);
    sum = block_sum(s, sm.redv);
  }
  if (tid == 0) {
    fc_rowstat r{};
    r.mx = mx;
    r.sum = sum;
    r.tau = unmono(tau_key);
    r.tie_idx = tie_idx;
    r.argmax = amax;
    sm.res = r;
    if (out) *out = r;
  }
  __syncthreads();
}

__device__ __forceinline__ float prob_at(const float* z, const fc_rowstat& rs, float T, int i) {
  return kept(z[i], i, mono(rs.tau), rs.tie_idx) ? expf(z[i] / T - rs.mx) / rs.sum : 0.f;
}

// Gumbel-max draw over V entries; mode 0: p, mode 1: residual max(0, p - q)
// renormalised (falls back to p when its mass is zero).
__device__ int block_draw(const float* __restrict__ zp, const fc_rowstat& sp, const float* __restrict__ zq,
                          const fc_rowstat& sq, int mode, float T, int V, uint64_t seed, int row, int rnd,
                          int slot, StatSmem& sm) {
  const int tid = threadIdx.x;
  float rsum = 0.f;
  if (mode == 1) {
    float s = 0.f;
    for (int i = tid; i < V; i += NTHR) s += fmaxf(prob_at(zp, sp, T, i) - prob_at(zq, sq, T, i), 0.f);
    rsum = block_sum(s, sm.redv);
    if (!(rsum > 0.f)) mode = 0;
  }
  const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  const int ngrp = (V + 3) >> 2;
  for (int gi = tid; gi < ngrp; gi += NTHR) {
    const u32x4 r = philox4x32_10(u32x4{(uint32_t)gi, (uint32_t)row, (uint32_t)rnd, (uint32_t)slot}, k0, k1);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int i = gi * 4 + w;
      if (i >= V) break;
      float p = prob_at(zp, sp, T, i);
      if (mode == 1) p = fmaxf(p - prob_at(zq, sq, T, i), 0.f) / rsum;
      const float sc = logf(fmaxf(p, 1e-10f)) + gumbel_of(pick(r, w));
      argmax_merge(bv, bi, sc, i);
    }
  }
  block_argmax(bv, bi, sm.redv, sm.redi);
  return bi;
}

__global__ __launch_bounds__(NTHR) void k_row_stats(const float* __restrict__ logits, int V, float T, int top_k,
                                                    fc_rowstat* __restrict__ stats) {
  __shared__ StatSmem sm;
  row_stats_block(logits + (int64_t)blockIdx.x * V, V, T, top_k, stats + blockIdx.x, sm);
}

int fc_launch_row_stats(const float* logits, int rows, int V, float T, int top_k, fc_rowstat* stats, hipStream_t s) {
  if (rows <= 0) return FC_OK;
  hipLaunchKernelGGL(k_row_stats, dim3(rows), dim3(NTHR), 0, s, logits, V, T, top_k, stats);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int32_t fc_row_stats(const float* logits, int32_t rows, int32_t V, float temperature, int32_t top_k,
                                fc_rowstat* stats, void* stream) {
  FC_CHECK_ARG(logits && stats && V > 0, "arguments");
  return fc_launch_row_stats(logits, rows, V, temperature, top_k, stats, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Speculative round kernels
// ---------------------------------------------------------------------------
struct SpecDev {  // the fc_spec_state fields the kernels read, by value
  int B, k, max_tokens, gen_cap, V;
  float T;
  int top_k;
  uint64_t seed;
  int *t_len, *d_len, *t_pend, *d_pend, *t_pend_n, *d_pend_n, *t_dirty, *d_dirty, *gen, *gen_n, *prompt_len,
      *round, *stall, *result;
  int *tok_d0, *off_d0, *start_d, *tok_ds, *off_ds, *tok_v, *off_v, *start_v, *drafts;
  float *q_logits, *p_logits;
  fc_rowstat *q_stats, *p_stats;
};

static SpecDev to_dev(const fc_spec_state* s) {
  SpecDev d;
  d.B = s->batch; d.k = s->k; d.max_tokens = s->max_tokens; d.gen_cap = s->gen_cap; d.V = s->vocab;
  d.T = s->temperature; d.top_k = s->top_k; d.seed = s->seed;
  d.t_len = s->t_len; d.d_len = s->d_len; d.t_pend = s->t_pend; d.d_pend = s->d_pend;
  d.t_pend_n = s->t_pend_n; d.d_pend_n = s->d_pend_n; d.t_dirty = s->t_dirty; d.d_dirty = s->d_dirty;
  d.gen = s->gen; d.gen_n = s->gen_n; d.prompt_len = s->prompt_len; d.round = s->round; d.stall = s->stall;
  d.result = s->result;
  d.tok_d0 = s->tok_d0; d.off_d0 = s->off_d0; d.start_d = s->start_d; d.tok_ds = s->tok_ds; d.off_ds = s->off_ds;
  d.tok_v = s->tok_v; d.off_v = s->off_v; d.start_v = s->start_v; d.drafts = s->drafts;
  d.q_logits = s->q_logits; d.p_logits = s->p_logits; d.q_stats = s->q_stats; d.p_stats = s->p_stats;
  return d;
}

__device__ __forceinline__ bool row_finished(const SpecDev& s, int b) {
  return s.gen_n[b] - s.prompt_len[b] >= s.max_tokens;
}

// Exclusive scan over the block (blockDim.x == PLAN_THR) of three counts
// per thread; returns the block totals. `carry` holds the running totals of
// earlier chunks of rows.
#define PLAN_THR 1024
__device__ __forceinline__ void scan3(int v[3], int tot[3], int* sm) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int x[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    x[q] = v[q];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x[q], o, WAVE);
      if (lane >= o) x[q] += y;
    }
  }
  __syncthreads();
  if (lane == 63)
#pragma unroll
    for (int q = 0; q < 3; ++q) sm[q * 16 + w] = x[q];
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    int before = 0, all = 0;
    for (int i = 0; i < PLAN_THR / 64; ++i) {
      const int t = sm[q * 16 + i];
      if (i < w) before += t;
      all += t;
    }
    v[q] = before + x[q] - v[q];  // exclusive prefix
    tot[q] = all;
  }
}

// Round plan (one workgroup): packed chunks for draft step 0 (the row's
// pending draft tokens), draft steps 1..k-1 (one token per active row) and
// the verify pass (pending target tokens then the k drafts, which the draft
// samplers write in place). Finished rows get no tokens. A stalled row
// (rollback backlog longer than FC_PMAX) drafts nothing: it re-feeds the next
// FC_PMAX tokens of each model's backlog gen[len, gen_n - 1) at draft step 0
// and in the verify chunk, until both caches hold everything before gen_n - 1.
__global__ __launch_bounds__(PLAN_THR) void k_spec_plan(SpecDev s) {
  __shared__ int sm[48];
  const int P = FC_PMAX, K = s.k, B = s.B;
  int carry[3] = {0, 0, 0};
  for (int b0 = 0; b0 < B; b0 += PLAN_THR) {
    const int b = b0 + threadIdx.x;
    const bool in = b < B;
    const bool live = in && !row_finished(s, b);
    const bool refeed = live && s.stall[b];
    const bool active = live && !refeed;
    int dn = 0, tn = 0;
    const int* gen = s.gen + (int64_t)(in ? b : 0) * s.gen_cap;
    if (active) {
      dn = min(max(s.d_pend_n[b], 0), P);
      tn = min(max(s.t_pend_n[b], 0), P);
    } else if (refeed) {
      const int last = s.gen_n[b] - 1;
      dn = min(max(last - s.d_len[b], 0), P);
      tn = min(max(last - s.t_len[b], 0), P);
    }
    int v[3] = {dn, active ? 1 : 0, active ? tn + K : tn}, tot[3];
    scan3(v, tot, sm);
    if (in) {
      const int o0 = carry[0] + v[0], o1 = carry[1] + v[1], o2 = carry[2] + v[2];
      s.off_d0[b] = o0;
      s.off_ds[b] = o1;
      s.off_v[b] = o2;
      if (refeed) {
        for (int j = 0; j < dn; ++j) s.tok_d0[o0 + j] = gen[s.d_len[b] + j];
        for (int j = 0; j < tn; ++j) s.tok_v[o2 + j] = gen[s.t_len[b] + j];
      } else {
        for (int j = 0; j < dn; ++j) s.tok_d0[o0 + j] = s.d_pend[b * P + j];
        for (int j = 0; j < tn; ++j) s.tok_v[o2 + j] = s.t_pend[b * P + j];
      }
      const int dl = s.d_len[b];
      s.start_d[b] = dl;
      for (int i = 1; i < K; ++i) s.start_d[i * B + b] = dl + dn + i - 1;
      s.start_v[b] = s.t_len[b];
    }
#pragma unroll
    for (int q = 0; q < 3; ++q) carry[q] += tot[q];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    s.off_d0[B] = carry[0];
    s.off_ds[B] = carry[1];
    s.off_v[B] = carry[2];
  }
}

// Where draft step i's proposal for row b goes: the verify chunk and the
// next draft step's chunk (active rows only; inactive rows own no slots).
__device__ __forceinline__ void place_draft(const SpecDev& s, int b, int i, int tok) {
  s.drafts[b * s.k + i] = tok;
  const int a0 = s.off_ds[b];
  if (s.off_ds[b + 1] == a0) return;
  s.tok_v[s.off_v[b + 1] - s.k + i] = tok;
  if (i + 1 < s.k) s.tok_ds[(i + 1) * s.B + a0] = tok;
}

// Draft step i: statistics of the draft logits row, proposal d_{i+1}
// (flaxchat/engine.py:493-499), written where the next chunks read it.
__global__ __launch_bounds__(NTHR) void k_draft_sample(SpecDev s, int i) {
  __shared__ StatSmem sm;
  const int b = blockIdx.x;
  const float* z = s.q_logits + ((int64_t)b * s.k + i) * s.V;
  fc_rowstat* rs = s.q_stats + b * s.k + i;
  row_stats_block(z, s.V, s.T, s.top_k, rs, sm);
  int tok;
  const fc_rowstat st = sm.res;
  if (s.T > 0.f) tok = block_draw(z, st, z, st, 0, s.T, s.V, s.seed, b, s.round[b], i, sm);
  else tok = st.argmax;
  if (threadIdx.x == 0) place_draft(s, b, i, tok);
}

// Candidates of chunks 4 blockIdx.x + wave of logits row blockIdx.y, one
// wave per chunk (lane l holds entries TK_EPL l .. + TK_EPL - 1). With
// `draw`, the G of every entry (counter (entry / 4, row, round[row], slot)):
// kept with the candidates, and the largest among the rest.
__global__ __launch_bounds__(TK_THR) void k_topk_cand(const float* __restrict__ z0, int64_t row_stride, int V,
                                                      int top_k, int draw, uint64_t seed, const int* __restrict__ round,
                                                      int slot, int nch, TkChunk* __restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = blockIdx.x * (TK_THR / 64) + wave, r = blockIdx.y;
  if (c >= nch) return;  // the whole wave
  const float* z = z0 + (int64_t)r * row_stride;
  const int e0 = c * TK_CH + lane * TK_EPL;
  float v[TK_EPL];
  bool ok[TK_EPL];
  int idx[TK_EPL];
  const bool vec = ((uintptr_t)z % 16 == 0) && e0 + TK_EPL - 1 < V;
#pragma unroll
  for (int q = 0; q < TK_EPL; q += 4) {
    if (vec) {
      const float4 t = *(const float4*)(z + e0 + q);
      v[q] = t.x; v[q + 1] = t.y; v[q + 2] = t.z; v[q + 3] = t.w;
    } else {
#pragma unroll
      for (int w = 0; w < 4; ++w) v[q + w] = e0 + q + w < V ? z[e0 + q + w] : -INFINITY;
    }
  }
#pragma unroll
  for (int q = 0; q < TK_EPL; ++q) {
    ok[q] = e0 + q < V;
    idx[q] = e0 + q;
  }
  const int kk = min(top_k, V - c * TK_CH);
  uint32_t key[TK_EPL];
  uint32_t lmax = 0u;
  bool lhas = false;
#pragma unroll
  for (int q = 0; q < TK_EPL; ++q) {
    key[q] = mono(v[q]);
    if (ok[q]) {
      lmax = max(lmax, key[q]);
      lhas = true;
    }
  }
  const uint32_t kmax = wave_max_u32(lmax);
  // lower bound for the chunk's kk-th largest key: the kk-th largest of the
  // lanes' maxima (kk entries reach it); the entries at or above it are few
  // for real logits and are searched narrowly, two per lane
  uint32_t tlo = 0u;
  if (wave_count(lhas) >= kk) {
    const uint32_t lk[1] = {lmax};
    const bool lo1[1] = {lhas};
    int unused;
    tlo = wave_kth_key<1>(lk, lo1, kk, 0u, kmax, unused);
  }
  int cnt = 0;
#pragma unroll
  for (int q = 0; q < TK_EPL; ++q) cnt += ok[q] && key[q] >= tlo;
  static_assert(TK_EPL < 32, "per-lane counts below 2^5");
  const int total = wave_sum_small<5>(cnt);
  int ngt;
  uint32_t tau;
  if (total <= TK_NARROW_WAVE) {
    __shared__ uint32_t cs[TK_THR / 64][TK_NARROW_WAVE];
    int p = wave_excl_small<5>(cnt);
#pragma unroll
    for (int q = 0; q < TK_EPL; ++q)
      if (ok[q] && key[q] >= tlo) cs[wave][p++] = key[q];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t k2[2] = {cs[wave][lane], cs[wave][lane + 64]};
    const bool o2[2] = {lane < total, lane + 64 < total};
    tau = wave_kth_key<2>(k2, o2, kk, tlo, kmax, ngt);
  } else {
    tau = wave_kth_key<TK_EPL>(key, ok, kk, 0u, kmax, ngt);
  }
  bool in[TK_EPL];
  wave_keep<TK_EPL>(key, ok, idx, tau, kk - ngt, in, nullptr);
  int nin = 0;
#pragma unroll
  for (int q = 0; q < TK_EPL; ++q) nin += in[q];
  int pos = wave_excl_small<5>(nin);
  TkChunk* o = out + (int64_t)r * nch + c;
  float bg = -INFINITY;
  int bgi = 0x7fffffff;
  const int rnd = draw ? round[r] : 0;
#pragma unroll
  for (int q = 0; q < TK_EPL; q += 4) {
    u32x4 rr = {0u, 0u, 0u, 0u};
    if (draw)
      rr = philox4x32_10(u32x4{(uint32_t)((e0 + q) >> 2), (uint32_t)r, (uint32_t)rnd, (uint32_t)slot},
                         (uint32_t)seed, (uint32_t)(seed >> 32));
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float G = draw ? gumbel_of(pick(rr, w)) : 0.f;
      if (in[q + w]) {
        o->z[pos] = v[q + w];
        o->idx[pos] = e0 + q + w;
        o->gz[pos] = G;
        ++pos;
      } else if (draw && ok[q + w]) {
        argmax_merge(bg, bgi, G, e0 + q + w);
      }
    }
  }
  wave_argmax(bg, bgi);
  if (lane == 0) {
    o->g = bg;
    o->gi = bgi;
    o->n = kk;
    o->kmax = kmax;
  }
}

__global__ __launch_bounds__(TK_THR) void k_topk_draft(SpecDev s, int i, const TkChunk* __restrict__ ch, int nch) {
  const int b = blockIdx.x;
  const TkRow r = tk_finish_row(ch + (int64_t)b * nch, nch, s.V, s.top_k, s.T, true);
  if (threadIdx.x == 0) {
    s.q_stats[b * s.k + i] = r.st;
    place_draft(s, b, i, r.tok);
  }
}

// Statistics of each logits row (the target's k+1 rows per row), one workgroup per row.
__global__ __launch_bounds__(TK_THR) void k_topk_stats(const TkChunk* __restrict__ ch, int nch, int rows, int V,
                                                       int top_k, float T, fc_rowstat* __restrict__ stats) {
  const int r = blockIdx.x;
  const TkRow t = tk_finish_row(ch + (int64_t)r * nch, nch, V, top_k, T, false);
  if (threadIdx.x == 0) stats[r] = t.st;
}

static bool tk_fast(const fc_spec_state* st) {
  return st->top_k > 0 && st->top_k <= TK_MAX && (st->vocab + TK_CH - 1) / TK_CH <= TK_NCH;
}
static int tk_nch(int V) { return (V + TK_CH - 1) / TK_CH; }

// The rollback state machine after one accept/reject pass: append the
// emitted tokens, move the cache lengths and pending tokens of both models,
// and fill the row's result record.
__device__ void bookkeep(const SpecDev& s, int b, const int* emitted, int n_emit, int acc, int rej,
                         int bonus_emitted, int kp, int rnd) {
  int* res = s.result + (int64_t)b * FC_RES_STRIDE;
  const int K = s.k;
  const int G0 = s.gen_n[b];
  int* gen = s.gen + (int64_t)b * s.gen_cap;
  int flags = 0;
  for (int i = 0; i < n_emit; ++i)
    if (G0 + i < s.gen_cap) gen[G0 + i] = emitted[i];
  const int gn = min(G0 + n_emit, s.gen_cap);
  s.gen_n[b] = gn;
  const int P = FC_PMAX;
  const int tb = s.t_len[b], npt = s.t_pend_n[b], db = s.d_len[b], npd = s.d_pend_n[b];
  if (bonus_emitted) {
    const int bonus = emitted[n_emit - 1];
    s.t_len[b] = tb + npt + kp;
    s.t_pend[b * P] = bonus;
    s.t_pend_n[b] = 1;
    if (kp == K) {
      s.d_len[b] = db + npd + K - 1;
      s.d_pend[b * P] = s.drafts[b * K + K - 1];
      s.d_pend[b * P + 1] = bonus;
      s.d_pend_n[b] = 2;
    } else {
      s.d_len[b] = db + npd + kp;
      s.d_pend[b * P] = bonus;
      s.d_pend_n[b] = 1;
    }
    if (rej >= 0) {  // rejected last draft: caches keep it, output has the correction
      const int pos = G0 + kp - 1;
      s.t_dirty[b] = min(s.t_dirty[b], pos);
      s.d_dirty[b] = min(s.d_dirty[b], pos);
    }
  } else {
    // roll back to the accept point, or to the stale entry if earlier; the
    // tokens from there on are fed again next round (the reference
    // re-prefills both models from scratch here, engine.py:593-606)
    const int a = acc;
    const int t_new = min(s.t_dirty[b], tb + npt + a - 1);
    const int d_new = min(s.d_dirty[b], db + npd + a - 1);
    s.t_dirty[b] = BIG_POS;
    s.d_dirty[b] = BIG_POS;
    const int tp = gn - t_new, dp = gn - d_new;
    s.t_len[b] = t_new;
    s.d_len[b] = d_new;
    if (tp <= P && dp <= P) {
      for (int i = 0; i < tp; ++i) s.t_pend[b * P + i] = gen[t_new + i];
      s.t_pend_n[b] = tp;
      for (int i = 0; i < dp; ++i) s.d_pend[b * P + i] = gen[d_new + i];
      s.d_pend_n[b] = dp;
    } else {  // the next rounds re-feed gen[len, gn-1) of both models (k_spec_plan)
      s.t_pend[b * P] = gen[gn - 1];
      s.t_pend_n[b] = 1;
      s.d_pend[b * P] = gen[gn - 1];
      s.d_pend_n[b] = 1;
      flags |= 1;
      s.stall[b] = 1;
    }
  }
  if (gn - s.prompt_len[b] >= s.max_tokens) flags |= 4;
  s.round[b] = rnd + 1;
  res[0] = n_emit;
  res[1] = acc;
  res[2] = rej;
  res[3] = flags;
  res[4] = kp;
  res[5] = s.t_pend_n[b];
  res[6] = s.d_pend_n[b];
  for (int i = 0; i < n_emit && i < FC_RES_STRIDE - 8; ++i) res[8 + i] = emitted[i];
}

// Accept/reject decision of one row (flaxchat/engine.py:525-592) from the
// target row statistics `ps` (k+1 rows) and the draft statistics: accepted
// drafts, the greedy correction and greedy bonus go to `emitted`; a sampled
// rejection or bonus is left as a draw request (mode / bonus_draw).
struct Decision {
  int mode;        // -1 finished, -2 stalled (re-feeding), 0 no rejection draw, 1 draw from p, 2 from the residual
  int row;         // verify row of the rejection draw
  int n, acc, rej, bonus, kp;
  int bonus_draw;  // the bonus token is still to be drawn (sampling)
  int emitted[24];
};
static_assert(sizeof(Decision) == 32 * sizeof(int), "Decision layout");

// mode -1: the row finished; -2: the row is stalled (it re-fed rollback
// backlog this round and drafted nothing).
// The sampled acceptance test's inputs for draft position i (p and q of the
// draft token, the uniform), which k_accept_decide's lanes load for every
// position at once (pre != nullptr) instead of one position after another.
struct AcceptIn {
  float pm, pd;
  double u;
};
__device__ __forceinline__ AcceptIn accept_in(const SpecDev& s, int b, const fc_rowstat* ps, int i) {
  const int K = s.k, V = s.V;
  // positions past the row's drafts this round hold older values; clamped so
  // every load stays in the row (decide reads only the row's own positions)
  const int dt = min(max(s.drafts[b * K + i], 0), V - 1);
  const fc_rowstat qs = s.q_stats[b * K + i];
  const float* zp = s.p_logits + ((int64_t)b * (K + 1) + i) * V;
  const float* zq = s.q_logits + ((int64_t)b * K + i) * V;
  AcceptIn a;
  a.pm = prob_at(zp, ps[i], s.T, dt);
  a.pd = prob_at(zq, qs, s.T, dt);
  const u32x4 r = philox4x32_10(u32x4{0u, (uint32_t)b, (uint32_t)s.round[b], (uint32_t)(SLOT_ACCEPT + i)},
                                (uint32_t)s.seed, (uint32_t)(s.seed >> 32));
  a.u = (double)u_half(r.x);
  return a;
}

__device__ void decide(const SpecDev& s, int b, const fc_rowstat* ps, Decision& d,
                       const AcceptIn* pre = nullptr) {
  const int K = s.k, V = s.V;
  const bool greedy = !(s.T > 0.f);
  const int ng = s.gen_n[b] - s.prompt_len[b];
  const int kp = min(K, s.max_tokens - ng);
  d.kp = kp;
  d.mode = -1;
  d.row = 0;
  d.n = 0;
  d.acc = 0;
  d.rej = -1;
  d.bonus = 0;
  d.bonus_draw = 0;
  if (kp <= 0) return;
  if (s.stall[b]) {
    d.mode = -2;
    d.kp = 0;
    return;
  }
  d.mode = 0;
  int acc = 0, n = 0;
  for (int i = 0; i < kp; ++i) {
    const int dt = s.drafts[b * K + i];
    if (greedy) {
      const int am = ps[i].argmax;
      d.emitted[n++] = am;
      ++acc;
      if (am != dt) { d.rej = i; break; }
    } else {
      const AcceptIn a = pre != nullptr ? pre[i] : accept_in(s, b, ps, i);
      const float pm = a.pm, pd = a.pd;
      if (pd == 0.f) {
        d.mode = 1; d.row = i; ++acc; d.rej = i;
        break;
      }
      const double ap = fmin(1.0, (double)pm / (double)pd);
      const double u = a.u;
      if (u < ap) {
        d.emitted[n++] = dt;
        ++acc;
      } else {
        d.mode = 2; d.row = i; ++acc; d.rej = i;
        break;
      }
    }
  }
  d.acc = acc;
  d.bonus = acc == kp;
  if (d.bonus) {
    if (greedy) d.emitted[n++] = ps[kp].argmax;
    else d.bonus_draw = 1;
  }
  d.n = n;
}

// A finished row (flag 4) or a stalled row that re-fed part of its backlog
// this round (flag 8): the caches grew by the tokens k_spec_plan fed; once
// both hold everything before gen_n - 1, the row resumes with that token
// pending in each model (FC_PMAX-sized pending lists are exact from then on).
// The round counter of a stalled row does not move, so its random stream
// does not depend on how many rounds the re-feed takes.
__device__ void idle_row(const SpecDev& s, int b, int mode) {
  int* res = s.result + (int64_t)b * FC_RES_STRIDE;
  if (mode == -2) {
    const int last = s.gen_n[b] - 1;
    s.d_len[b] += s.off_d0[b + 1] - s.off_d0[b];
    s.t_len[b] += s.off_v[b + 1] - s.off_v[b];  // a stalled row has no drafts in the verify chunk
    if (s.d_len[b] >= last && s.t_len[b] >= last) s.stall[b] = 0;
  }
  res[0] = 0; res[1] = 0; res[2] = -1; res[3] = mode == -2 ? 8 : 4; res[4] = 0;
  res[5] = s.t_pend_n[b]; res[6] = s.d_pend_n[b];
  if (mode != -2) s.round[b] += 1;
}

// Accept/reject with the top-k filter (one workgroup per row): decision,
// rejection / bonus draws, rollback bookkeeping.
__global__ __launch_bounds__(NTHR) void k_accept(SpecDev s) {
  __shared__ StatSmem sm;
  __shared__ Decision d;
  const int b = blockIdx.x, tid = threadIdx.x;
  const int K = s.k, V = s.V;
  if (tid == 0) decide(s, b, s.p_stats + b * (K + 1), d);
  __syncthreads();
  if (d.mode < 0) {
    if (tid == 0) idle_row(s, b, d.mode);
    return;
  }
  const int rnd = s.round[b];
  if (d.mode > 0) {
    const int i = d.row;
    const fc_rowstat ps = s.p_stats[b * (K + 1) + i];
    const fc_rowstat qs = s.q_stats[b * K + i];
    const int c = block_draw(s.p_logits + ((int64_t)b * (K + 1) + i) * V, ps, s.q_logits + ((int64_t)b * K + i) * V,
                             qs, d.mode == 2 ? 1 : 0, s.T, V, s.seed, b, rnd, SLOT_REJECT, sm);
    if (tid == 0) d.emitted[d.n++] = c;
    __syncthreads();
  }
  if (d.bonus_draw) {
    const int kp = d.kp;
    const fc_rowstat ps = s.p_stats[b * (K + 1) + kp];
    const int bt = block_draw(s.p_logits + ((int64_t)b * (K + 1) + kp) * V, ps, nullptr, ps, 0, s.T, V, s.seed, b,
                              rnd, SLOT_BONUS, sm);
    if (tid == 0) d.emitted[d.n++] = bt;
    __syncthreads();
  }
  if (tid != 0) return;
  bookkeep(s, b, d.emitted, d.n, d.acc, d.rej, d.bonus, d.kp, rnd);
}

// ---------------------------------------------------------------------------
// Vocab passes without a top-k filter, split over many workgroups: a logits
// row is cut into chunks of VP_CHUNK * NV entries (one 256-thread workgroup,
// 4 consecutive entries per thread and sub-block, so one Philox block per
// thread), each writes a 32-byte partial, and one wave per row merges them.
//
// A Gumbel-max draw over log(max(p, 1e-10)) + G with p = exp(x - M) / S,
// x = z / T, is taken in one pass before M and S are known: per element the
// score is max(x - C, log 1e-10) + G with C = M + log S, so per chunk it is
//   max(a_c - (M - m_c + log S), log 1e-10 + g_c),
// a_c = max(x - m_c + G) (relative to the chunk's max m_c, which keeps the
// sums small for any T), g_c = max G; the argmax index of each term is kept.
// ---------------------------------------------------------------------------
#define VP_THR 256
#define VP_CHUNK (VP_THR * 4)
// workgroup budget of a vocab pass: rows x chunks (of VP_CHUNK * nv entries)
// stays within it, nv <= 8. 8192 puts cfg4's 224 verify rows on 32 chunks
// each instead of 8 (4.796-4.799 vs 4.802-4.807 ms per round, alternating
// builds); draft rows (32 x 64 chunks) are unchanged.
#ifndef VP_MAXWG
#define VP_MAXWG 8192
#endif

struct DPart {  // one chunk of a draw from finished row statistics
  float sc; int si;      // max of log(max(p, 1e-10)) + G
  float A; int Ai;       // residual: max of log r + G over r = max(p - q, 0) > 0
  float g; int gi;       // max of G
  float R; int pad;      // residual: sum of r
};
static_assert(sizeof(VPart) == 32 && sizeof(DPart) == 32, "partial layout");


// Four entries e..e+3 of row z (-inf beyond V).
__device__ __forceinline__ void load4(const float* __restrict__ z, int e, int V, bool vec, float* v) {
  if (vec && e + 3 < V) {
    const float4 q = *reinterpret_cast<const float4*>(z + e);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else {
#pragma unroll
    for (int w = 0; w < 4; ++w) v[w] = e + w < V ? z[e + w] : -INFINITY;
  }
}

// Block-wide (value, index) argmax for a VP_THR block; result in every thread.
__device__ __forceinline__ void vp_argmax(float& v, int& i, float* redv, int* redi) {
  block_argmax(v, i, redv, redi);
}

// Two block-wide argmaxes through one LDS exchange (redv / redi hold 2 x the
// wave count); each result equals what vp_argmax returns for it.
__device__ __forceinline__ void vp_argmax2(float& v, int& i, float& u, int& j, float* redv, int* redi) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = VP_THR / 64;
  wave_argmax(v, i);
  wave_argmax(u, j);
  __syncthreads();
  if (lane == 0) {
    redv[w] = v;
    redi[w] = i;
    redv[nw + w] = u;
    redi[nw + w] = j;
  }
  __syncthreads();
  float bv = redv[0], bu = redv[nw];
  int bi = redi[0], bj = redi[nw];
  for (int k = 1; k < nw; ++k) {
    argmax_merge(bv, bi, redv[k], redi[k]);
    argmax_merge(bu, bj, redv[nw + k], redi[nw + k]);
  }
  v = bv;
  i = bi;
  u = bu;
  j = bj;
}

// Chunk partials of rows r of z0 (row stride `row_stride` floats): argmax,
// max / exp-sum of z/T (T > 0), and with `draw` the Gumbel-max terms of the
// draw with counter (element / 4, r, round[r], slot).
template <int NV>
__global__ __launch_bounds__(VP_THR) void k_vpart(const float* __restrict__ z0, int64_t row_stride, int V, float T,
                                                  int vec, int draw, uint64_t seed, const int* __restrict__ round,
                                                  int slot, VPart* __restrict__ out) {
  __shared__ float redv[16];
  __shared__ int redi[16];
  const int c = blockIdx.x, r = blockIdx.y, tid = threadIdx.x;
  const float* z = z0 + (int64_t)r * row_stride;
  float v[NV][4];
  int e0[NV];
  float bz = -INFINITY;
  int bzi = 0x7fffffff;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    e0[j] = (c * NV + j) * VP_CHUNK + tid * 4;
    load4(z, e0[j], V, vec != 0, v[j]);
#pragma unroll
    for (int w = 0; w < 4; ++w)
      if (e0[j] + w < V) argmax_merge(bz, bzi, v[j][w], e0[j] + w);
  }
  vp_argmax(bz, bzi, redv, redi);
  VPart p;
  p.zmax = bz;
  p.zarg = bzi;
  p.m = 0.f;
  p.s = 1.f;
  p.a = -INFINITY;
  p.ai = 0x7fffffff;
  p.g = -INFINITY;
  p.gi = 0x7fffffff;
  if (T > 0.f) {
    // max of z / T is max(z) / T exactly (division by T > 0 is monotone
    // under round-to-nearest), so the argmax reduction above gives it
    const float m = bz / T;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int w = 0; w < 4; ++w) v[j][w] = v[j][w] / T;
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int w = 0; w < 4; ++w)
        if (e0[j] + w < V) sum += expf(v[j][w] - m);
    sum = block_sum(sum, redv);
    p.m = m;
    p.s = sum;
    if (draw) {
      const int rnd = round[r];
      float ba = -INFINITY, bg = -INFINITY;
      int bai = 0x7fffffff, bgi = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        if (e0[j] >= V) continue;
        const u32x4 rr = philox4x32_10(u32x4{(uint32_t)(e0[j] >> 2), (uint32_t)r, (uint32_t)rnd, (uint32_t)slot},
                                       (uint32_t)seed, (uint32_t)(seed >> 32));
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int i = e0[j] + w;
          if (i >= V) break;
          const float G = gumbel_of(pick(rr, w));
          argmax_merge(ba, bai, (v[j][w] - m) + G, i);
          argmax_merge(bg, bgi, G, i);
        }
      }
      vp_argmax2(ba, bai, bg, bgi, redv, redi);
      p.a = ba;
      p.ai = bai;
      p.g = bg;
      p.gi = bgi;
    }
  }
  if (tid == 0) out[(int64_t)r * gridDim.x + c] = p;
}

static int vp_nv(int rows, int V) {
  int nv = 1;
  while (nv < 8 && (int64_t)rows * ((V + VP_CHUNK * nv - 1) / (VP_CHUNK * nv)) > VP_MAXWG) nv *= 2;
  return nv;
}
static int vp_nch(int V, int nv) { return (V + VP_CHUNK * nv - 1) / (VP_CHUNK * nv); }

static int launch_vpart(const float* z0, int64_t row_stride, int rows, int V, float T, bool draw, uint64_t seed,
                        const int* round, int slot, VPart* out, int* nch_out, hipStream_t s) {
  const int nv = vp_nv(rows, V), nch = vp_nch(V, nv);
  const int vec = (V % 4 == 0) && (row_stride % 4 == 0) && ((uintptr_t)z0 % 16 == 0);
  const dim3 grid(nch, rows);
  switch (nv) {
    case 1: hipLaunchKernelGGL(k_vpart<1>, grid, dim3(VP_THR), 0, s, z0, row_stride, V, T, vec, (int)draw, seed, round, slot, out); break;
    case 2: hipLaunchKernelGGL(k_vpart<2>, grid, dim3(VP_THR), 0, s, z0, row_stride, V, T, vec, (int)draw, seed, round, slot, out); break;
    case 4: hipLaunchKernelGGL(k_vpart<4>, grid, dim3(VP_THR), 0, s, z0, row_stride, V, T, vec, (int)draw, seed, round, slot, out); break;
    default: hipLaunchKernelGGL(k_vpart<8>, grid, dim3(VP_THR), 0, s, z0, row_stride, V, T, vec, (int)draw, seed, round, slot, out); break;
  }
  FC_LAUNCH_CHECK();
  *nch_out = nch;
  return FC_OK;
}

// One wave merges the nch partials of a row: statistics and (with `draw`)
// the winner of the row's draw.
__device__ RowMerge wave_merge_row(const VPart* __restrict__ p, int nch, bool samp, bool draw) {
  const int lane = threadIdx.x & 63;
  float M = -INFINITY, zm = -INFINITY;
  int zi = 0x7fffffff;
  for (int c = lane; c < nch; c += 64) {
    M = fmaxf(M, p[c].m);
    argmax_merge(zm, zi, p[c].zmax, p[c].zarg);
  }
  M = wave_max(M);
  wave_argmax(zm, zi);
  RowMerge rm;
  rm.argmax = zi;
  rm.M = 0.f;
  rm.S = 1.f;
  rm.tok = zi;
  if (!samp) return rm;
  float S = 0.f;
  for (int c = lane; c < nch; c += 64) S += p[c].s * expf(p[c].m - M);
  S = wave_sum(S);
  rm.M = M;
  rm.S = S;
  if (draw) {
    const float lS = logf(S), lf = log_floor();
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int c = lane; c < nch; c += 64) {
      argmax_merge(bv, bi, p[c].a - ((M - p[c].m) + lS), p[c].ai);
      argmax_merge(bv, bi, lf + p[c].g, p[c].gi);
    }
    wave_argmax(bv, bi);
    rm.tok = bi;
  }
  return rm;
}

// Draft step i without top-k: merge of the step's partials (one wave per row),
// proposal d_{i+1} written where the next chunks read it.
__global__ __launch_bounds__(VP_THR) void k_draft_finish(SpecDev s, int i, const VPart* __restrict__ part,
                                                         int nch) {
  const int b = blockIdx.x * (VP_THR / 64) + (threadIdx.x >> 6);
  if (b >= s.B) return;
  const bool samp = s.T > 0.f;
  const RowMerge rm = wave_merge_row(part + (int64_t)b * nch, nch, samp, samp);
  if ((threadIdx.x & 63) == 0) {
    s.q_stats[b * s.k + i] = make_rowstat(rm, s.V);
    place_draft(s, b, i, rm.tok);
  }
}

// Draft step i when the logits GEMM wrote the partials (one per column tile):
// one workgroup per row.
#ifndef FC_DRAFT_VP_FUSE
#define FC_DRAFT_VP_FUSE 1
#endif
#ifndef FC_DRAFT_MERGE_IN_EMBED
#define FC_DRAFT_MERGE_IN_EMBED 1
#endif
static_assert(VP_THR == FC_VOCAB_THR, "the merge's workgroup size");
__global__ __launch_bounds__(VP_THR) void k_draft_finish_wide(DraftMerge dm) { draft_merge_row(dm, blockIdx.x); }

// The DraftMerge of draft step i's partials (one per column tile, nch a row)
static DraftMerge draft_merge(const SpecDev& d, int i, const VPart* part, int nch) {
  DraftMerge dm{};
  dm.part = part;
  dm.nch = nch;
  dm.q_stats = d.q_stats;
  dm.drafts = d.drafts;
  dm.tok_v = d.tok_v;
  dm.off_v = d.off_v;
  dm.off_ds = d.off_ds;
  dm.tok_ds = d.tok_ds;
  dm.B = d.B;
  dm.k = d.k;
  dm.V = d.V;
  dm.step = i;
  dm.T = d.T;
  return dm;
}

// Verify rows without top-k: merge the k+1 rows' partials into p_stats,
// decide, and record the draw requests for k_draw_part.
__global__ __launch_bounds__(VP_THR) void k_accept_decide(SpecDev s, const VPart* __restrict__ part, int nch,
                                                          Decision* __restrict__ ctl) {
  __shared__ fc_rowstat ps[FC_PMAX + 1];
  __shared__ Decision d;
  const int b = blockIdx.x, w = threadIdx.x >> 6;
  const int R = s.k + 1;
  const bool samp = s.T > 0.f;
  for (int j = w; j < R; j += VP_THR / 64) {
    const RowMerge rm = wave_merge_row(part + ((int64_t)b * R + j) * nch, nch, samp, false);
    if ((threadIdx.x & 63) == 0) {
      const fc_rowstat rs = make_rowstat(rm, s.V);
      ps[j] = rs;
      s.p_stats[b * R + j] = rs;
    }
  }
  __syncthreads();
  __shared__ AcceptIn pre[FC_PMAX];
  if (s.T > 0.f && threadIdx.x < min(s.k, FC_PMAX)) pre[threadIdx.x] = accept_in(s, b, ps, threadIdx.x);
  __syncthreads();
  if (threadIdx.x != 0) return;
  decide(s, b, ps, d, s.k <= FC_PMAX ? pre : nullptr);
  ctl[b] = d;
}

// Top-k rows (T > 0): the decisions from the finished target row statistics
// (k_topk_stats), recorded for k_draw_part / k_accept_finish like
// k_accept_decide's; one thread per row.
__global__ __launch_bounds__(64) void k_accept_decide_st(SpecDev s, Decision* __restrict__ ctl) {
  __shared__ Decision d;
  const int b = blockIdx.x;
  if (threadIdx.x != 0) return;
  decide(s, b, s.p_stats + b * (s.k + 1), d);
  ctl[b] = d;
}

// Chunk partials of the rejection draw (z = 0, slot 48, from p or from the
// residual max(0, p - q)) and the bonus draw (z = 1, slot 49, from p) of
// each row, as requested by k_accept_decide (k_accept_decide_st). TOPK: p
// and q are zero outside the rows' keep sets (the statistics' tau / tie_idx).
template <int NV, bool TOPK>
__global__ __launch_bounds__(VP_THR) void k_draw_part(SpecDev s, const Decision* __restrict__ ctl, int vec,
                                                      DPart* __restrict__ out) {
  __shared__ float redv[16];
  __shared__ int redi[16];
  const int c = blockIdx.x, b = blockIdx.y, q = blockIdx.z, tid = threadIdx.x;
  const Decision& d = ctl[b];
  int mode, row, slot;
  if (q == 0) {
    mode = d.mode > 0 ? d.mode : 0;
    row = d.row;
    slot = SLOT_REJECT;
  } else {
    mode = d.bonus_draw ? 1 : 0;
    row = d.kp;
    slot = SLOT_BONUS;
  }
  if (mode == 0) return;  // uniform over the block
  const int K = s.k, V = s.V;
  const float T = s.T;
  const float* zp = s.p_logits + ((int64_t)b * (K + 1) + row) * V;
  const fc_rowstat ps = s.p_stats[b * (K + 1) + row];
  const float* zq = s.q_logits + ((int64_t)b * K + min(row, K - 1)) * V;
  const fc_rowstat qs = s.q_stats[b * K + min(row, K - 1)];
  const int rnd = s.round[b];
  const uint32_t tp = TOPK ? mono(ps.tau) : 0u, tq = TOPK ? mono(qs.tau) : 0u;
  float bs = -INFINITY, bA = -INFINITY, bg = -INFINITY, R = 0.f;
  int bsi = 0x7fffffff, bAi = 0x7fffffff, bgi = 0x7fffffff;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int e = (c * NV + j) * VP_CHUNK + tid * 4;
    if (e >= V) continue;
    float vp[4], vq[4];
    load4(zp, e, V, vec != 0, vp);
    if (mode == 2) load4(zq, e, V, vec != 0, vq);
    const u32x4 rr = philox4x32_10(u32x4{(uint32_t)(e >> 2), (uint32_t)b, (uint32_t)rnd, (uint32_t)slot},
                                   (uint32_t)s.seed, (uint32_t)(s.seed >> 32));
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int i = e + w;
      if (i >= V) break;
      const float G = gumbel_of(pick(rr, w));
      float p = expf(vp[w] / T - ps.mx) / ps.sum;
      if (TOPK && !kept(vp[w], i, tp, ps.tie_idx)) p = 0.f;
      argmax_merge(bs, bsi, logf(fmaxf(p, 1e-10f)) + G, i);
      if (mode == 2) {
        float pq = expf(vq[w] / T - qs.mx) / qs.sum;
        if (TOPK && !kept(vq[w], i, tq, qs.tie_idx)) pq = 0.f;
        const float rv = fmaxf(p - pq, 0.f);
        R += rv;
        if (rv > 0.f) argmax_merge(bA, bAi, logf(rv) + G, i);
        argmax_merge(bg, bgi, G, i);
      }
    }
  }
  vp_argmax(bs, bsi, redv, redi);
  DPart o;
  o.sc = bs;
  o.si = bsi;
  o.A = -INFINITY;
  o.Ai = 0x7fffffff;
  o.g = -INFINITY;
  o.gi = 0x7fffffff;
  o.R = 0.f;
  o.pad = 0;
  if (mode == 2) {
    vp_argmax(bA, bAi, redv, redi);
    vp_argmax(bg, bgi, redv, redi);
    R = block_sum(R, redv);
    o.A = bA;
    o.Ai = bAi;
    o.g = bg;
    o.gi = bgi;
    o.R = R;
  }
  if (tid == 0) out[((int64_t)b * 2 + q) * gridDim.x + c] = o;
}

// Winner of one draw from its chunk partials (one wave): the residual
// max(0, p - q) renormalised when its mass is positive, else p.
__device__ int wave_merge_draw(const DPart* __restrict__ p, int nch, bool residual) {
  const int lane = threadIdx.x & 63;
  float R = 0.f;
  if (residual) {
    for (int c = lane; c < nch; c += 64) R += p[c].R;
    R = wave_sum(R);
  }
  const bool use_r = residual && R > 0.f;
  const float lR = use_r ? logf(R) : 0.f, lf = log_floor();
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int c = lane; c < nch; c += 64) {
    if (use_r) {
      argmax_merge(bv, bi, p[c].A - lR, p[c].Ai);
      argmax_merge(bv, bi, lf + p[c].g, p[c].gi);
    } else {
      argmax_merge(bv, bi, p[c].sc, p[c].si);
    }
  }
  wave_argmax(bv, bi);
  return bi;
}

// Rejection / bonus tokens from the draw partials, then the bookkeeping.
__global__ __launch_bounds__(64) void k_accept_finish(SpecDev s, const Decision* __restrict__ ctl,
                                                      const DPart* __restrict__ part, int nch) {
  __shared__ int em[32];
  const int b = blockIdx.x;
  const Decision* d = ctl + b;
  const int mode = d->mode, bonus_draw = d->bonus_draw;
  if (mode < 0) {
    if (threadIdx.x == 0) idle_row(s, b, mode);
    return;
  }
  int trej = -1, tbonus = -1;
  if (mode > 0) trej = wave_merge_draw(part + (int64_t)b * 2 * nch, nch, mode == 2);
  if (bonus_draw) tbonus = wave_merge_draw(part + ((int64_t)b * 2 + 1) * nch, nch, false);
  if (threadIdx.x != 0) return;
  int n = d->n;
  for (int i = 0; i < n; ++i) em[i] = d->emitted[i];
  if (mode > 0) em[n++] = trej;
  if (bonus_draw) em[n++] = tbonus;
  bookkeep(s, b, em, n, d->acc, d->rej, d->bonus, d->kp, s.round[b]);
}

// Layout of fc_spec_state.part: Decision[B] | VPart[B*(k+1)][nch1] | DPart[B][2][nch1],
// nch1 = chunks per row at NV = 1 (the most any pass uses).
struct PartLayout {
  Decision* ctl;
  VPart* vp;
  DPart* dp;
  TkChunk* tk;  // top-k candidates of up to batch x (k + 1) rows
  int64_t bytes;
  int64_t vp_cap;  // VParts at vp
};
static PartLayout part_layout(void* base, int B, int K, int V) {
  const int64_t nch1 = vp_nch(V, 1);
  PartLayout L;
  // VParts: the k + 1 verify rows' chunks, or one per 64-column tile of a
  // draft step's logits row (vocab padded to a multiple of 64) when its
  // logits GEMM writes them
  L.vp_cap = (int64_t)B * std::max((int64_t)(K + 1) * nch1, (int64_t)(V + 63) / 64);
  const int64_t o_vp = fc_align((int64_t)B * sizeof(Decision));
  const int64_t o_dp = o_vp + fc_align(L.vp_cap * (int64_t)sizeof(VPart));
  const int64_t o_tk = o_dp + fc_align((int64_t)B * 2 * nch1 * sizeof(DPart));
  L.bytes = o_tk + fc_align((int64_t)B * (K + 1) * tk_nch(V) * sizeof(TkChunk));
  char* p = (char*)base;
  L.ctl = (Decision*)p;
  L.vp = (VPart*)(p + o_vp);
  L.dp = (DPart*)(p + o_dp);
  L.tk = (TkChunk*)(p + o_tk);
  return L;
}

extern "C" int64_t fc_spec_part_bytes(int32_t batch, int32_t k, int32_t vocab) {
  if (batch <= 0 || k <= 0 || vocab <= 0) return -1;
  return part_layout(nullptr, batch, k, vocab).bytes;
}

// The chunked passes serve rows without a top-k filter (and greedy rows: the
// top-k set does not move the argmax); the filtered case keeps one
// workgroup per row for its radix select.
static bool chunked(const fc_spec_state* st) {
  return !(st->temperature > 0.f) || st->top_k <= 0 || st->top_k >= st->vocab;
}

static int check_spec(const fc_spec_state* st) {
  FC_CHECK_ARG(st && st->batch > 0 && st->k > 0 && st->k <= 16 && st->vocab > 0, "spec state sizes (k in 1..16)");
  FC_CHECK_ARG(st->t_len && st->d_len && st->t_pend && st->d_pend && st->t_pend_n && st->d_pend_n &&
                   st->t_dirty && st->d_dirty && st->gen && st->gen_n && st->prompt_len && st->round && st->stall &&
                   st->result && st->q_logits && st->p_logits && st->q_stats && st->p_stats && st->drafts &&
                   st->tok_v && st->off_v && st->start_v && st->tok_ds && st->off_ds && st->tok_d0 && st->off_d0 &&
                   st->start_d && st->part,
               "spec state pointers");
  FC_CHECK_ARG(st->part_bytes >= fc_spec_part_bytes(st->batch, st->k, st->vocab),
               "part_bytes below fc_spec_part_bytes(batch, k, vocab)");
  return FC_OK;
}

extern "C" int32_t fc_spec_accept(const fc_spec_state* st, void* stream) {
  int rc = check_spec(st);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  SpecDev d = to_dev(st);
  const int B = st->batch, K = st->k, V = st->vocab;
  if (!chunked(st)) {
    if (tk_fast(st)) {  // the target rows' keep sets from per-chunk candidates
      const PartLayout L = part_layout(st->part, B, K, V);
      const int nc = tk_nch(V);
      hipLaunchKernelGGL(k_topk_cand, dim3((nc + 3) / 4, B * (K + 1)), dim3(TK_THR), 0, s, st->p_logits, (int64_t)V,
                         V, st->top_k, 0, st->seed, st->round, 0, nc, L.tk);
      FC_LAUNCH_CHECK();
      hipLaunchKernelGGL(k_topk_stats, dim3(B * (K + 1)), dim3(TK_THR), 0, s, L.tk, nc, B * (K + 1), V,
                         st->top_k, st->temperature, st->p_stats);
      FC_LAUNCH_CHECK();
    } else {
      rc = fc_launch_row_stats(st->p_logits, B * (K + 1), V, st->temperature, st->top_k, st->p_stats, s);
      if (rc) return rc;
    }
    if (!tk_fast(st)) {
      hipLaunchKernelGGL(k_accept, dim3(B), dim3(NTHR), 0, s, d);
      FC_LAUNCH_CHECK();
      return FC_OK;
    }
    // decisions from the statistics, the draws split over the vocabulary
    const PartLayout L = part_layout(st->part, B, K, V);
    hipLaunchKernelGGL(k_accept_decide_st, dim3(B), dim3(64), 0, s, d, L.ctl);
    FC_LAUNCH_CHECK();
  } else {
    const PartLayout L = part_layout(st->part, B, K, V);
    int nch = 0;
    rc = launch_vpart(st->p_logits, V, B * (K + 1), V, st->temperature, false, st->seed, st->round, 0, L.vp, &nch,
                      s);
    if (rc) return rc;
    hipLaunchKernelGGL(k_accept_decide, dim3(B), dim3(VP_THR), 0, s, d, L.vp, nch, L.ctl);
    FC_LAUNCH_CHECK();
  }
  const PartLayout L = part_layout(st->part, B, K, V);
  const int nv = vp_nv(B, V), dch = vp_nch(V, nv);
  const int vec = (V % 4 == 0) && ((uintptr_t)st->p_logits % 16 == 0) && ((uintptr_t)st->q_logits % 16 == 0);
  const dim3 grid(dch, B, 2);
  const bool tk = !chunked(st);
#define DRAW_PART(NVV)                                                                                       \
  {                                                                                                          \
    if (tk) hipLaunchKernelGGL((k_draw_part<NVV, true>), grid, dim3(VP_THR), 0, s, d, L.ctl, vec, L.dp);      \
    else hipLaunchKernelGGL((k_draw_part<NVV, false>), grid, dim3(VP_THR), 0, s, d, L.ctl, vec, L.dp);        \
  }
  switch (nv) {
    case 1: DRAW_PART(1); break;
    case 2: DRAW_PART(2); break;
    case 4: DRAW_PART(4); break;
    default: DRAW_PART(8); break;
  }
#undef DRAW_PART
  FC_LAUNCH_CHECK();
  hipLaunchKernelGGL(k_accept_finish, dim3(B), dim3(64), 0, s, d, L.ctl, L.dp, dch);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

// Chunk capacities of a round (per row: FC_PMAX pending draft tokens at
// step 0; FC_PMAX pending target tokens + k drafts at verify) and the token
// counts the kernel shapes are tuned for.
struct RoundChunks {
  fc_chunk d0, ds, v;
};
static RoundChunks round_chunks(const fc_spec_state* st) {
  const int B = st->batch, K = st->k, V = st->vocab;
  RoundChunks r{};
  r.d0.max_tokens = B * FC_PMAX;
  r.d0.max_per_row = FC_PMAX;
  r.d0.typ_tokens = 2 * B;
  r.d0.tokens = st->tok_d0;
  r.d0.row_off = st->off_d0;
  r.d0.start = st->start_d;
  r.d0.n_out = 1;
  r.d0.logits = st->q_logits;
  r.d0.logits_stride = (int64_t)K * V;
  r.ds = r.d0;
  r.ds.max_tokens = B;
  r.ds.max_per_row = 1;
  r.ds.typ_tokens = B;
  r.ds.row_off = st->off_ds;
  r.v.max_tokens = B * (FC_PMAX + K);
  r.v.max_per_row = FC_PMAX + K;
  r.v.typ_tokens = B * (K + 2);
  r.v.tokens = st->tok_v;
  r.v.row_off = st->off_v;
  r.v.start = st->start_v;
  r.v.n_out = K + 1;
  r.v.logits = st->p_logits;
  r.v.logits_stride = (int64_t)(K + 1) * V;
  return r;
}

extern "C" int64_t fc_spec_workspace_bytes(const fc_model* target, const fc_model* draft, int32_t batch,
                                           int32_t k) {
  if (!target || !draft || batch <= 0 || k <= 0 || k > 16) return -1;
  const int B = batch;
  int64_t a = fc_forward_workspace_bytes(target, B, B * (FC_PMAX + k), FC_PMAX + k, B * (k + 2));
  int64_t b = fc_forward_workspace_bytes(draft, B, B * FC_PMAX, FC_PMAX, 2 * B);
  int64_t c = fc_forward_workspace_bytes(draft, B, B, 1, B);
  if (a < 0 || b < 0 || c < 0) return -1;
  return std::max(a, std::max(b, c));
}

extern "C" int32_t fc_spec_round(const fc_model* target, const fc_cache* tcache, const fc_model* draft,
                                 const fc_cache* dcache, const fc_spec_state* st, void* work, int64_t work_bytes,
                                 void* stream) {
  int rc = check_spec(st);
  if (rc) return rc;
  FC_CHECK_ARG(target && draft && tcache && dcache, "models / caches");
  FC_CHECK_ARG(target->vocab == draft->vocab && target->vocab == st->vocab, "main and draft vocab differ");
  FC_CHECK_ARG(tcache->batch == st->batch && dcache->batch == st->batch, "batch");
  hipStream_t s = (hipStream_t)stream;
  SpecDev d = to_dev(st);
  const int B = st->batch, K = st->k, V = st->vocab;
  hipLaunchKernelGGL(k_spec_plan, dim3(1), dim3(PLAN_THR), 0, s, d);
  FC_LAUNCH_CHECK();
  const bool fast = chunked(st);
  const PartLayout L = part_layout(st->part, B, K, V);
  const RoundChunks rcn = round_chunks(st);
  int pend_merge = 0;  // partials per row of the previous draft step still to merge
  for (int i = 0; i < K; ++i) {
    fc_chunk ch = i == 0 ? rcn.d0 : rcn.ds;
    if (i > 0) {
      ch.tokens = st->tok_ds + (int64_t)i * B;
      ch.start = st->start_d + (int64_t)i * B;
    }
    ch.logits = st->q_logits + (int64_t)i * V;
    // without top-k the draft's logits GEMM also writes the vocab-pass
    // partials where its kernel can (one per 64 / 128-column tile; Philox
    // counter row = batch row b, as in the separate pass)
    VocabFuse vf{};
    if (fast && FC_DRAFT_VP_FUSE) {
      vf.vp = L.vp;
      vf.vp_cap = L.vp_cap;
      vf.max_tiles = VP_THR * VP_WIDE_MAXP;
      vf.T = st->temperature;
      vf.draw = st->temperature > 0.f;
      vf.slot = i;
      vf.seed = st->seed;
      vf.round = st->round;
    }
    // the previous step's partials, merged by this step's embedding kernel
    DraftMerge dmg{};
    if (pend_merge > 0) dmg = draft_merge(d, i - 1, L.vp, pend_merge);
    int fused = 0;
    rc = fc_forward_vp(draft, dcache, &ch, work, work_bytes, stream, fast ? &vf : nullptr, &fused,
                       pend_merge > 0 ? &dmg : nullptr);
    if (rc) return rc;
    pend_merge = 0;
    if (fast && fused > 0) {
      // the next draft step's chunk (one token per row) merges them in its
      // embedding kernel; the last step's go to the verify chunk through the
      // merge kernel
      if (FC_DRAFT_MERGE_IN_EMBED && i + 1 < K && fc_embed_merges(draft, &rcn.ds)) pend_merge = fused;
      else hipLaunchKernelGGL(k_draft_finish_wide, dim3(B), dim3(VP_THR), 0, s, draft_merge(d, i, L.vp, fused));
    } else if (fast) {
      int nch = 0;
      rc = launch_vpart(st->q_logits + (int64_t)i * V, (int64_t)K * V, B, V, st->temperature, st->temperature > 0.f,
                        st->seed, st->round, i, L.vp, &nch, s);
      if (rc) return rc;
      if (FC_DRAFT_MERGE_IN_EMBED && i + 1 < K && fc_embed_merges(draft, &rcn.ds) &&
          nch <= VP_THR * VP_WIDE_MAXP) {  // the separate pass's chunks, merged the same way
        pend_merge = nch;
      } else {
        hipLaunchKernelGGL(k_draft_finish, dim3((B + 3) / 4), dim3(VP_THR), 0, s, d, i, L.vp, nch);
      }
    } else if (tk_fast(st)) {  // top-k: per-chunk candidates, then one workgroup per row
      const int nc = tk_nch(V);
      hipLaunchKernelGGL(k_topk_cand, dim3((nc + 3) / 4, B), dim3(TK_THR), 0, s, st->q_logits + (int64_t)i * V,
                         (int64_t)K * V, V, st->top_k, 1, st->seed, st->round, i, nc, L.tk);
      FC_LAUNCH_CHECK();
      hipLaunchKernelGGL(k_topk_draft, dim3(B), dim3(TK_THR), 0, s, d, i, L.tk, nc);
    } else {
      hipLaunchKernelGGL(k_draft_sample, dim3(B), dim3(NTHR), 0, s, d, i);
    }
    FC_LAUNCH_CHECK();
  }
  fc_chunk vch = rcn.v;
  rc = fc_forward(target, tcache, &vch, work, work_bytes, stream);
  if (rc) return rc;
  return fc_spec_accept(st, stream);
}

// ---------------------------------------------------------------------------
// generate_fast sampling step (flaxchat/engine.py:308-324, 343-368) and
// Engine.generate's per-step token choice (flaxchat/engine.py:666-683, 773-790)
// ---------------------------------------------------------------------------
// ENGINE = false: rows stop on eos or at max_pos (done[] / max_pos[]).
// ENGINE = true: no stop (completion is decided by the caller); a row with
// forced[b] >= 0 takes that token instead of a sample.
template <bool ENGINE>
__global__ __launch_bounds__(NTHR) void k_fast_sample(const float* __restrict__ logits, int V, float T, int top_k,
                                                      uint64_t seed, int eos, int* __restrict__ gen, int gen_cap,
                                                      int* __restrict__ pos, int* __restrict__ done,
                                                      int* __restrict__ step, const int* __restrict__ max_pos,
                                                      const int* __restrict__ forced, int* __restrict__ tok_cur,
                                                      fc_rowstat* __restrict__ stats) {
  __shared__ StatSmem sm;
  const int b = blockIdx.x;
  int tok = -1;
  if (ENGINE) {
    tok = forced[b];
  } else if (done[b] || pos[b] >= max_pos[b]) {
    return;
  }
  if (tok < 0) {
    const float* z = logits + (int64_t)b * V;
    row_stats_block(z, V, T, top_k, stats + b, sm);
    const fc_rowstat rs = sm.res;
    if (T > 0.f) {
      const uint32_t tk = mono(rs.tau);
      const int rnd = step[b];
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      const int ngrp = (V + 3) >> 2;
      for (int gi = threadIdx.x; gi < ngrp; gi += NTHR) {
        const u32x4 r = philox4x32_10(u32x4{(uint32_t)gi, (uint32_t)b, (uint32_t)rnd, 0u}, (uint32_t)seed,
                                      (uint32_t)(seed >> 32));
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int i = gi * 4 + w;
          if (i >= V) break;
          if (!kept(z[i], i, tk, rs.tie_idx)) continue;
          argmax_merge(bv, bi, z[i] / T + gumbel_of(pick(r, w)), i);
        }
      }
      block_argmax(bv, bi, sm.redv, sm.redi);
      tok = bi;
    } else {
      tok = rs.argmax;
    }
  }
  if (threadIdx.x == 0) {
    const int p = pos[b] + 1;
    if (p < gen_cap) gen[(int64_t)b * gen_cap + p] = tok;
    pos[b] = p;
    tok_cur[b] = tok;
    step[b] += 1;
    if (!ENGINE && tok == eos) done[b] = 1;
  }
}

extern "C" int32_t fc_fast_sample(const float* logits, int32_t batch, int32_t V, float temperature, int32_t top_k,
                                  uint64_t seed, int32_t eos, int32_t* gen, int32_t gen_cap, int32_t* pos,
                                  int32_t* done, int32_t* step, const int32_t* max_pos, int32_t* tok_cur,
                                  fc_rowstat* stats, void* stream) {
  FC_CHECK_ARG(logits && gen && pos && done && step && max_pos && tok_cur && stats, "null pointer");
  FC_CHECK_ARG(batch > 0 && V > 0 && gen_cap > 0, "sizes");
  hipLaunchKernelGGL(k_fast_sample<false>, dim3(batch), dim3(NTHR), 0, (hipStream_t)stream, logits, V, temperature,
                     top_k, seed, eos, gen, gen_cap, pos, done, step, max_pos, nullptr, tok_cur, stats);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int32_t fc_engine_sample(const float* logits, int32_t batch, int32_t V, float temperature, int32_t top_k,
                                    uint64_t seed, const int32_t* forced, int32_t* gen, int32_t gen_cap, int32_t* pos,
                                    int32_t* step, int32_t* tok_cur, fc_rowstat* stats, void* stream) {
  FC_CHECK_ARG(logits && forced && gen && pos && step && tok_cur && stats, "null pointer");
  FC_CHECK_ARG(batch > 0 && V > 0 && gen_cap > 0, "sizes");
  hipLaunchKernelGGL(k_fast_sample<true>, dim3(batch), dim3(NTHR), 0, (hipStream_t)stream, logits, V, temperature,
                     top_k, seed, -1, gen, gen_cap, pos, nullptr, step, nullptr, forced, tok_cur, stats);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

// ---------------------------------------------------------------------------
// Cross-entropy of the full-sequence forward (flaxchat/gpt.py:446-452):
// one workgroup per logits row, max then sum of exp (fixed reduction order)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_cross_entropy(const float* __restrict__ logits, int64_t row_stride,
                                                       const int* __restrict__ targets, int V,
                                                       float* __restrict__ loss) {
  __shared__ float red[16];
  const int r = blockIdx.x;
  const int t = targets[r];
  if (t < 0 || t >= V) {  // masked rows (the caller keeps t < V)
    if (threadIdx.x == 0) loss[r] = 0.f;
    return;
  }
  const float* z = logits + (int64_t)r * row_stride;
  float mx = -INFINITY;
  for (int i = threadIdx.x; i < V; i += blockDim.x) mx = fmaxf(mx, z[i]);
  mx = block_max(mx, red);
  float s = 0.f;
  for (int i = threadIdx.x; i < V; i += blockDim.x) s += expf(z[i] - mx);
  s = block_sum(s, red);
  if (threadIdx.x == 0) loss[r] = (mx + logf(s)) - z[t];
}

extern "C" int32_t fc_cross_entropy(const float* logits, int64_t row_stride, const int32_t* targets, int32_t rows,
                                    int32_t V, float* loss, void* stream) {
  FC_CHECK_ARG(logits && targets && loss, "null pointer");
  FC_CHECK_ARG(rows >= 0 && V > 0 && row_stride >= V, "sizes");
  if (rows == 0) return FC_OK;
  hipLaunchKernelGGL(k_cross_entropy, dim3(rows), dim3(256), 0, (hipStream_t)stream, logits, row_stride, targets, V,
                     loss);
  FC_LAUNCH_CHECK();
  return FC_OK;
}
