// Per-row merge of vocab-pass partials by one 256-thread workgroup, shared by
// the draft step's finish kernel and the embedding kernel that can do that
// merge for the next draft step itself (fc_forward's DraftMerge).
#pragma once
#include "fc_common.h"
#include "fc_internal.h"

#define FC_VOCAB_THR 256
#define VP_WIDE_MAXP 4  // partials per thread: rows of up to 1024 partials

__device__ __forceinline__ float log_floor() { return logf(1e-10f); }

// A merged row: max of z / T and the exp-sum relative to it, the argmax, the drawn token.
struct RowMerge { float M, S; int argmax, tok; };

__device__ __forceinline__ fc_rowstat make_rowstat(const RowMerge& rm, int V) {
  fc_rowstat rs{};
  rs.mx = rm.M;
  rs.sum = rm.S;
  rs.tau = -INFINITY;
  rs.tie_idx = V;
  rs.argmax = rm.argmax;
  return rs;
}

// The merge of wave_merge_row by a whole workgroup, for rows of many
// partials (the logits GEMM's column tiles: up to FC_VOCAB_THR * MAXP): every
// thread loads its MAXP partials at once, then three block reductions in a
// fixed order.
template <int MAXP>
__device__ RowMerge block_merge_row(const VPart* __restrict__ p, int nch, bool samp, bool draw) {
  __shared__ float redv[2 * (FC_VOCAB_THR / 64)];
  __shared__ int redi[2 * (FC_VOCAB_THR / 64)];
  float4 lo[MAXP], hi[MAXP];
#pragma unroll
  for (int u = 0; u < MAXP; ++u) {
    const int c = threadIdx.x + u * FC_VOCAB_THR;
    if (c < nch) {
      const float4* src = reinterpret_cast<const float4*>(p + c);
      lo[u] = src[0];
      hi[u] = src[1];
    } else {
      lo[u] = make_float4(-INFINITY, __int_as_float(0x7fffffff), -INFINITY, 0.f);
      hi[u] = make_float4(-INFINITY, __int_as_float(0x7fffffff), -INFINITY, __int_as_float(0x7fffffff));
    }
  }
  float M = -INFINITY, zm = -INFINITY;
  int zi = 0x7fffffff;
#pragma unroll
  for (int u = 0; u < MAXP; ++u) {
    M = fmaxf(M, lo[u].z);
    argmax_merge(zm, zi, lo[u].x, __float_as_int(lo[u].y));
  }
  M = block_max(M, redv);
  block_argmax(zm, zi, redv, redi);
  RowMerge rm;
  rm.argmax = zi;
  rm.M = 0.f;
  rm.S = 1.f;
  rm.tok = zi;
  if (!samp) return rm;
  float S = 0.f;
#pragma unroll
  for (int u = 0; u < MAXP; ++u)
    if (lo[u].z != -INFINITY) S += lo[u].w * expf(lo[u].z - M);
  S = block_sum(S, redv);
  rm.M = M;
  rm.S = S;
  if (draw) {
    const float lS = logf(S), lf = log_floor();
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int u = 0; u < MAXP; ++u) {
      argmax_merge(bv, bi, hi[u].x - ((M - lo[u].z) + lS), __float_as_int(hi[u].y));
      argmax_merge(bv, bi, lf + hi[u].z, __float_as_int(hi[u].w));
    }
    block_argmax(bv, bi, redv, redi);
    rm.tok = bi;
  }
  return rm;
}

// Finish draft step `step` for row b (whole workgroup, every thread gets the
// token): merge the row's partials, record its statistics and the draft
// where the verify chunk and the next draft step read it (flaxchat/engine.py:
// 493-499; active rows only own chunk slots).
__device__ __forceinline__ int draft_merge_row(const DraftMerge& dm, int b) {
  const bool samp = dm.T > 0.f;
  const RowMerge rm = block_merge_row<VP_WIDE_MAXP>(dm.part + (int64_t)b * dm.nch, dm.nch, samp, samp);
  if (threadIdx.x == 0) {
    dm.q_stats[b * dm.k + dm.step] = make_rowstat(rm, dm.V);
    dm.drafts[b * dm.k + dm.step] = rm.tok;
    const int a0 = dm.off_ds[b];
    if (dm.off_ds[b + 1] != a0) {
      dm.tok_v[dm.off_v[b + 1] - dm.k + dm.step] = rm.tok;
      if (dm.step + 1 < dm.k) dm.tok_ds[(dm.step + 1) * dm.B + a0] = rm.tok;
    }
  }
  return rm.tok;
}
