// Chunked multi-token forward: embedding + smear, the transformer blocks and
// the softcapped head, on a preallocated KV cache.
//
// One call replaces `_single_step_forward` (flaxchat/engine.py:51-177) for
// every token of every row at once: the draft's 1-token steps, the target's
// (k+1)-token verify chunk and prompt prefill are the same code with a
// different chunk. Tokens are packed: row b feeds row_off[b+1] - row_off[b]
// tokens at consecutive positions from start[b], so rows with more pending
// tokens cost only their own tokens. The total is a device value; every
// kernel is launched for the capacity and work past the total exits.
// Activations between kernels (one row per packed token):
//   x, x0, xb   fp32 residual stream, x0 and the backout capture
//   h           RMS-normed GEMM input (model dtype)
//   qkv         fp32 projections, consumed by the prologue
//   q, y, hid   attention query / output and the ReLU^2 hidden (model dtype)
#include "fc_common.h"
#include "fc_internal.h"
#include "fc_vocab.h"

#define EMBED_MAXW 1024

// Eight consecutive entries of an embedding row as fp32.
__device__ __forceinline__ void ld8(const bf16_t* p, float* o) {
  const uint4 v = *(const uint4*)p;
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __uint_as_float(w[i] << 16);
    o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void ld8(const float* p, float* o) {
  const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}
__device__ __forceinline__ void st8(float* p, const float* v) {
  *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
  *(float4*)(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

// Embedding + RMSNorm + smear (flaxchat/engine.py:80-94), one workgroup per
// row. The smear chain x_t = n_t + g_t * x_{t-1} is sequential in t but
// elementwise in the model dimension: each thread owns 8 consecutive
// columns and walks the row's tokens, with the embedding loads of the next
// four tokens issued ahead of the dependent arithmetic. Also records the row
// and position of every packed token for the later per-token kernels.
//
// NORM (bf16, at most EMBED_NORM_MAX tokens per row, D <= 2048: one 8-column
// slice per thread): also the first layer's RMSNorm, h = x * rsqrt(mean(x^2)
// + 1e-6) in the next GEMM's fragment order, from per-token block sums of
// the new x kept in registers, which saves that layer's RMSNorm launch.
#define EMBED_AHEAD 4
#define EMBED_NORM_MAX 8
template <typename T, bool NORM>
__global__ __launch_bounds__(256) void k_embed(const T* __restrict__ wte, const float* __restrict__ smear_gate,
                                               float smear_lambda, float r0, float a0,
                                               const int* __restrict__ tokens, const int* __restrict__ row_off,
                                               const int* __restrict__ start, int max_per_row, int Mcap, int D,
                                               int cap, float* __restrict__ hist, float* __restrict__ x,
                                               float* __restrict__ x0, int* __restrict__ tok_row,
                                               int* __restrict__ tok_pos, int full_smear, bf16_t* __restrict__ h,
                                               DraftMerge dm) {
  __shared__ float sg[EMBED_MAXW], sinv[EMBED_MAXW];
  const int b = blockIdx.x;
  // NORM with dm.part: first finish the previous draft step for this row; its
  // draft is the row's one token here (written to tokens[] for the later
  // kernels by thread 0, so this kernel reads it from the merge, not memory)
  int merged = -1;
  if constexpr (NORM) {
    if (dm.part != nullptr) merged = draft_merge_row(dm, b);
  }
  const RowSpan sp = row_span(row_off, b, max_per_row, Mcap);
  const int base = sp.base, n = sp.n, s0 = start[b];
  if (n <= 0 || s0 < 0) {
    // a rejected row is empty: its packed slots (clamped to the capacity)
    // get row -1, which the attention prologue and the fused QKV epilogue
    // skip, so no stale index from an earlier chunk can write a cache row
    const int lo = max(row_off[b], 0), hi = min(row_off[b + 1], Mcap);
    for (int j = lo + (int)threadIdx.x; j < hi; j += blockDim.x) tok_row[j] = -1;
    return;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int j = threadIdx.x; j < n; j += blockDim.x) {
    tok_row[base + j] = b;
    tok_pos[base + j] = s0 + j;
  }
  // per token: 1 / rms of the embedding row and the smear gate
  for (int j = wave; j < n; j += 4) {
    const T* e = wte + (int64_t)(merged >= 0 ? merged : tokens[base + j]) * D;
    float ss = 0.f;
    for (int d = lane * 8; d < D; d += 64 * 8) {
      float v[8];
      ld8(e + d, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
    }
    ss = wave_sum(ss);
    const float inv = 1.f / sqrtf(ss / (float)D + 1e-6f);
    const float z = wave_sum(lane < 24 ? (ld<T>(e, lane) * inv) * smear_gate[lane] : 0.f);
    if (lane == 0) {
      sinv[j] = inv;
      sg[j] = smear_lambda * (1.f / (1.f + expf(-z)));
    }
  }
  __syncthreads();
  if constexpr (NORM) {
    __shared__ float nred[EMBED_NORM_MAX][4];
    const int c0 = threadIdx.x * 8;
    const bool act = c0 < D;
    float keep[EMBED_NORM_MAX][8], ssj[EMBED_NORM_MAX];
    float prev[8];
#pragma unroll
    for (int j = 0; j < EMBED_NORM_MAX; ++j) ssj[j] = 0.f;
    if (act) {
      if (s0 > 0) ld8(hist + ((int64_t)b * cap + s0 - 1) * D + c0, prev);
      else
#pragma unroll
        for (int i = 0; i < 8; ++i) prev[i] = 0.f;
      float ev[EMBED_NORM_MAX][8];
#pragma unroll
      for (int j = 0; j < EMBED_NORM_MAX; ++j)
        if (j < n) ld8(wte + (int64_t)(merged >= 0 ? merged : tokens[base + j]) * D + c0, ev[j]);
#pragma unroll
      for (int j = 0; j < EMBED_NORM_MAX; ++j) {
        if (j < n) {
          float xv[8], nv[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            nv[i] = ev[j][i] * sinv[j];
            xv[i] = nv[i] + sg[j] * prev[i];
            keep[j][i] = r0 * xv[i] + a0 * xv[i];
            ssj[j] += keep[j][i] * keep[j][i];
            prev[i] = full_smear ? nv[i] : xv[i];
          }
          const int pos = s0 + j;
          if (pos < cap) st8(hist + ((int64_t)b * cap + pos) * D + c0, prev);
          const int64_t m = base + j;
          st8(x0 + m * D + c0, xv);
          st8(x + m * D + c0, keep[j]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < EMBED_NORM_MAX; ++j) {
      const float t = wave_sum(ssj[j]);
      if (lane == 0) nred[j][wave] = t;
    }
    __syncthreads();
    if (act) {
#pragma unroll
      for (int j = 0; j < EMBED_NORM_MAX; ++j) {
        if (j < n) {
          const float ss = nred[j][0] + nred[j][1] + nred[j][2] + nred[j][3];
          const float inv = 1.f / sqrtf(ss / (float)D + 1e-6f);
          uint4 pk;
          pk.x = (uint32_t)f2bf(keep[j][0] * inv) | ((uint32_t)f2bf(keep[j][1] * inv) << 16);
          pk.y = (uint32_t)f2bf(keep[j][2] * inv) | ((uint32_t)f2bf(keep[j][3] * inv) << 16);
          pk.z = (uint32_t)f2bf(keep[j][4] * inv) | ((uint32_t)f2bf(keep[j][5] * inv) << 16);
          pk.w = (uint32_t)f2bf(keep[j][6] * inv) | ((uint32_t)f2bf(keep[j][7] * inv) << 16);
          *(uint4*)(h + frag_idx(base + j, c0, D)) = pk;  // 8 consecutive k: 16 contiguous bytes
        }
      }
    }
    return;
  }
  for (int c0 = threadIdx.x * 8; c0 < D; c0 += blockDim.x * 8) {
    float prev[8];
    if (s0 > 0) ld8(hist + ((int64_t)b * cap + s0 - 1) * D + c0, prev);
    else
#pragma unroll
      for (int i = 0; i < 8; ++i) prev[i] = 0.f;
    for (int j0 = 0; j0 < n; j0 += EMBED_AHEAD) {
      float ev[EMBED_AHEAD][8];
#pragma unroll
      for (int u = 0; u < EMBED_AHEAD; ++u) {
        const int j = min(j0 + u, n - 1);
        ld8(wte + (int64_t)tokens[base + j] * D + c0, ev[u]);
      }
#pragma unroll
      for (int u = 0; u < EMBED_AHEAD; ++u) {
        const int j = j0 + u;
        if (j < n) {
          float xv[8], xr[8], nv[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            nv[i] = ev[u][i] * sinv[j];
            xv[i] = nv[i] + sg[j] * prev[i];
            xr[i] = r0 * xv[i] + a0 * xv[i];
            prev[i] = full_smear ? nv[i] : xv[i];  // GPT.__call__ smears with n_{t-1}, decode with x_{t-1}
          }
          const int pos = s0 + j;
          if (pos < cap) st8(hist + ((int64_t)b * cap + pos) * D + c0, prev);
          const int64_t m = base + j;
          st8(x0 + m * D + c0, xv);
          st8(x + m * D + c0, xr);
        }
      }
    }
  }
}

// A residual-stream update left pending by a split-K GEMM: the S partial
// products in part[S][rows][D] still have to be added to x, with the
// epilogue of that GEMM (EPI_ADD: x += y; EPI_MLPOUT: residual add, backout
// capture, then the next layer's lambda mix or the final backout).
struct Pending {
  int S, mode, rows;
  const float* part;
  const float* x0;
  float* xb;
  float r, a, lb;
  int capture, last;
};

// h = x * rsqrt(mean(x^2) + 1e-6) (flaxchat/gpt.py:44-46), after applying a
// pending update to x. n_out == 0: one workgroup per packed token (rows past
// the device total *Mdev exit). n_out > 0 (the head): output row
// b * n_out + r normalises the token row_off[b+1] - n_out + r, the r-th of
// row b's last n_out tokens; the residual stream is dead after it, so the
// finished x is not stored back (a row with fewer than n_out tokens reads a
// clamped row and its logits are unspecified).
#define NORM_MAXV 4  // float4 per thread: D <= 4096
template <typename TO>
__global__ __launch_bounds__(256) void k_rmsnorm(float* __restrict__ x, TO* __restrict__ h, int D, int Mcap,
                                                 const int* __restrict__ Mdev, const int* __restrict__ row_off,
                                                 int n_out, Pending p) {
  __shared__ float red[16];
  const int row = blockIdx.x, tid = threadIdx.x;
  int64_t in_row = row;
  if (n_out > 0) {
    const int b = row / n_out, r = row - b * n_out;
    in_row = min(max(row_off[b + 1] - n_out + r, 0), Mcap - 1);
  } else if (Mdev != nullptr && row >= *Mdev) {
    return;
  }
  const bool store_x = n_out == 0;
  const int D4 = D >> 2;
  float4* xr = (float4*)(x + in_row * D);
  float4 v[NORM_MAXV];
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < NORM_MAXV; ++u) {
    const int i = tid + 256 * u;
    if (i < D4) {
      float4 t = xr[i];
      if (p.S > 0) {
        // all split partials of this float4 are loaded together, summed in order
        float4 pp[FC_MAX_SPLIT];
#pragma unroll
        for (int s = 0; s < FC_MAX_SPLIT; ++s)
          if (s < p.S) pp[s] = ((const float4*)(p.part + ((int64_t)s * p.rows + in_row) * D))[i];
#pragma unroll
        for (int s = 0; s < FC_MAX_SPLIT; ++s)
          if (s < p.S) {
            t.x += pp[s].x; t.y += pp[s].y; t.z += pp[s].z; t.w += pp[s].w;
          }
        if (p.mode == EPI_MLPOUT) {
          const int64_t o = in_row * D4 + i;
          float4 xb_v = {0.f, 0.f, 0.f, 0.f};
          if (p.capture) {
            ((float4*)p.xb)[o] = t;
            xb_v = t;
          } else if (p.last) {
            xb_v = ((const float4*)p.xb)[o];
          }
          if (p.last) {
            t.x = t.x - p.lb * xb_v.x; t.y = t.y - p.lb * xb_v.y;
            t.z = t.z - p.lb * xb_v.z; t.w = t.w - p.lb * xb_v.w;
          } else {
            const float4 z = ((const float4*)p.x0)[o];
            t.x = p.r * t.x + p.a * z.x; t.y = p.r * t.y + p.a * z.y;
            t.z = p.r * t.z + p.a * z.z; t.w = p.r * t.w + p.a * z.w;
          }
        }
        if (store_x) xr[i] = t;
      }
      v[u] = t;
      ss += t.x * t.x + t.y * t.y + t.z * t.z + t.w * t.w;
    }
  }
  ss = block_sum(ss, red);
  const float inv = 1.f / sqrtf(ss / (float)D + 1e-6f);
  // h is the next GEMM's operand: fragment order in bf16 (4 consecutive k
  // stay contiguous), row-major in fp32
#pragma unroll
  for (int u = 0; u < NORM_MAXV; ++u) {
    const int i = tid + 256 * u;
    if (i < D4) {
      const int64_t o = act_idx<TO>(row, 4 * i, D);
      if constexpr (sizeof(TO) == 2) {
        uint2 pk;
        pk.x = (uint32_t)f2bf(v[u].x * inv) | ((uint32_t)f2bf(v[u].y * inv) << 16);
        pk.y = (uint32_t)f2bf(v[u].z * inv) | ((uint32_t)f2bf(v[u].w * inv) << 16);
        *(uint2*)(h + o) = pk;
      } else {
        *(float4*)(h + o) = make_float4(v[u].x * inv, v[u].y * inv, v[u].z * inv, v[u].w * inv);
      }
    }
  }
}

struct FwdWork {
  float *x, *x0, *xb, *qkv, *ssq;
  void *h, *q, *y, *hid, *part;
  int *tok_row, *tok_pos;
  int64_t part_bytes, total;
  GemmWork gw;
};

// Workspace layout for up to `max_tokens` packed tokens (`typ_tokens`
// typical) over `B` rows of at most `max_per_row` tokens.
static FwdWork carve(const fc_model* m, int B, int max_tokens, int max_per_row, int typ_tokens, char* base) {
  const int64_t M = max_tokens;
  const int D = m->n_embd, H = m->n_head, G = m->n_kv_head, hd = m->head_dim;
  const int es = m->dtype == FC_BF16 ? 2 : 4;
  FwdWork w{};
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    char* p = base ? base + off : nullptr;
    off += fc_align(bytes);
    return p;
  };
  w.x = (float*)take(M * D * 4);
  w.x0 = (float*)take(M * D * 4);
  w.xb = (float*)take(M * D * 4);
  w.qkv = (float*)take(M * (H + 2 * G) * hd * 4);
  const int64_t M16 = round16(M);  // GEMM operands in fragment order cover whole 16-row blocks
  w.h = take(M16 * D * es);
  w.q = take(M * H * hd * es);
  w.y = take(M16 * H * hd * es);
  w.hid = take(M16 * 4 * D * es);
  w.ssq = (float*)take((int64_t)(D / 16) * M * 4);  // folded norm: per 16+ column tile and row
  w.tok_row = (int*)take(M * 4);
  w.tok_pos = (int*)take(M * 4);
  // attention splits are sized for the largest key range a cache can hold
  w.part_bytes = fc_attn_part_bytes(B, max_per_row, H, G, hd, 1 << 20);
  w.part = take(w.part_bytes);
  // split-K partials of the two GEMMs that write the residual stream
  int64_t gp = std::max(fc_gemm_part_bytes(typ_tokens, (int)M, D, H * hd, m->dtype),
                        fc_gemm_part_bytes(typ_tokens, (int)M, D, 4 * D, m->dtype));
  w.gw.part = (float*)take(gp);
  w.gw.part_bytes = gp;
  w.total = off;
  return w;
}

static int typ_of(int max_tokens, int typ_tokens) {
  return typ_tokens > 0 && typ_tokens <= max_tokens ? typ_tokens : max_tokens;
}

extern "C" int64_t fc_forward_workspace_bytes(const fc_model* m, int32_t batch, int32_t max_tokens,
                                              int32_t max_per_row, int32_t typ_tokens) {
  if (!m || batch <= 0 || max_tokens <= 0 || max_per_row <= 0) return -1;
  return carve(m, batch, max_tokens, max_per_row, typ_of(max_tokens, typ_tokens), nullptr).total;
}

static int check_model(const fc_model* m) {
  FC_CHECK_ARG(m && m->layers && m->wte && m->lm_head, "model pointers");
  FC_CHECK_ARG(m->dtype == FC_F32 || m->dtype == FC_BF16, "dtype");
  FC_CHECK_ARG(m->n_head > 0 && m->n_kv_head > 0 && m->n_head % m->n_kv_head == 0, "heads");
  FC_CHECK_ARG(m->head_dim * m->n_head == m->n_embd, "head_dim * n_head must equal n_embd");
  FC_CHECK_ARG(m->n_embd % 8 == 0 && m->n_embd >= 24 && m->n_embd <= 4096,
               "n_embd must be a multiple of 8 in [24, 4096]");
  FC_CHECK_ARG(m->vocab > 0 && m->vocab <= m->vocab_pad, "vocab");
  FC_CHECK_ARG(m->dtype != FC_BF16 || (m->n_embd % 64 == 0 && m->vocab_pad % 32 == 0),
               "bf16 needs n_embd % 64 == 0 and vocab_pad % 32 == 0 (fragment-order GEMM operands)");
  return FC_OK;
}

extern "C" int32_t fc_forward(const fc_model* m, const fc_cache* c, const fc_chunk* ch, void* work,
                              int64_t work_bytes, void* stream) {
  int nch = 0;
  return fc_forward_vp(m, c, ch, work, work_bytes, stream, nullptr, &nch);
}

// bf16 chunks of at most EMBED_NORM_MAX tokens per row (n_embd <= 2048): the
// embedding kernel also writes the first layer's RMSNorm output, and can
// finish the previous draft step (DraftMerge)
bool fc_embed_merges(const fc_model* m, const fc_chunk* ch) {
  return m->dtype == FC_BF16 && ch->max_per_row <= EMBED_NORM_MAX && m->n_embd <= 2048 && m->n_embd % 8 == 0;
}

int fc_forward_vp(const fc_model* m, const fc_cache* c, const fc_chunk* ch, void* work, int64_t work_bytes,
                  void* stream, const VocabFuse* vpf, int* nch, const DraftMerge* dm) {
  *nch = 0;
  int rc = check_model(m);
  if (rc) return rc;
  FC_CHECK_ARG(c && c->k && c->v && c->hist && c->batch > 0 && c->cap > 0 && c->cap % 32 == 0, "cache");
  FC_CHECK_ARG(ch && ch->tokens && ch->row_off && ch->start, "chunk pointers");
  FC_CHECK_ARG(ch->max_tokens > 0 && ch->max_per_row > 0 && ch->max_per_row <= EMBED_MAXW &&
                   ch->max_per_row <= ch->max_tokens,
               "chunk sizes (max_per_row in [1, 1024] and <= max_tokens)");
  FC_CHECK_ARG(ch->n_out >= 0 && ch->n_out <= ch->max_per_row, "n_out");
  FC_CHECK_ARG((int64_t)c->batch * ch->n_out <= ch->max_tokens, "batch * n_out must not exceed max_tokens");
  FC_CHECK_ARG(ch->n_out == 0 || ch->logits, "logits pointer");
  hipStream_t s = (hipStream_t)stream;
  const int B = c->batch, Mcap = ch->max_tokens, Mtyp = typ_of(Mcap, ch->typ_tokens);
  const int* Mdev = ch->row_off + B;
  const int D = m->n_embd, H = m->n_head, G = m->n_kv_head, hd = m->head_dim;
  const int NQKV = (H + 2 * G) * hd;
  FwdWork w = carve(m, B, Mcap, ch->max_per_row, Mtyp, (char*)work);
  FC_CHECK_ARG(work && work_bytes >= w.total, "forward workspace too small");
  const int dt = m->dtype;
  const int64_t layer_elems = (int64_t)B * G * c->cap * hd;
  const int es = dt == FC_BF16 ? 2 : 4;
  const int typ_per_row = std::max(1, (Mtyp + B - 1) / B);
  const bool fuse_qkv = fc_gemm_fuses_qkv(Mtyp, NQKV, D, dt, hd);
  // bf16: the RMSNorm between attention and MLP is folded into the GEMMs (the
  // attention c_proj keeps a bf16 copy of x and per-tile sums of squares,
  // c_fc scales its rows by 1 / rms); fp32 keeps the exact RMSNorm kernel
  const bool fold = dt == FC_BF16 && fc_gemm_fold_ok(Mtyp, D);
  FC_CHECK_ARG((ch->flags & ~FC_CHUNK_FULL_SMEAR) == 0, "unknown fc_chunk flags");
  const int full_smear = ch->flags & FC_CHUNK_FULL_SMEAR;

  // bf16 chunks of few tokens per row: the embedding kernel also writes the
  // first layer's RMSNorm output (h), and that layer's RMSNorm launch is skipped
  const bool embed_norm = fc_embed_merges(m, ch);
  // the previous draft step's merge, run by this chunk's embedding kernel
  FC_CHECK_ARG(dm == nullptr || (embed_norm && ch->max_per_row == 1 && dm->part && dm->nch > 0 &&
                                 dm->nch <= FC_VOCAB_THR * VP_WIDE_MAXP && dm->B == B),
               "draft merge: a one-token-per-row bf16 draft chunk, at most 1024 partials per row");
  const DraftMerge dmv = dm != nullptr ? *dm : DraftMerge{};
  if (embed_norm)
    hipLaunchKernelGGL((k_embed<bf16_t, true>), dim3(B), dim3(256), 0, s, (const bf16_t*)m->wte, m->smear_gate,
                       m->smear_lambda, m->layers[0].resid_lambda, m->layers[0].x0_lambda, ch->tokens, ch->row_off,
                       ch->start, ch->max_per_row, Mcap, D, c->cap, c->hist, w.x, w.x0, w.tok_row, w.tok_pos,
                       full_smear, (bf16_t*)w.h, dmv);
  else if (dt == FC_BF16)
    hipLaunchKernelGGL((k_embed<bf16_t, false>), dim3(B), dim3(256), 0, s, (const bf16_t*)m->wte, m->smear_gate,
                       m->smear_lambda, m->layers[0].resid_lambda, m->layers[0].x0_lambda, ch->tokens, ch->row_off,
                       ch->start, ch->max_per_row, Mcap, D, c->cap, c->hist, w.x, w.x0, w.tok_row, w.tok_pos,
                       full_smear, nullptr, DraftMerge{});
  else
    hipLaunchKernelGGL((k_embed<float, false>), dim3(B), dim3(256), 0, s, (const float*)m->wte, m->smear_gate,
                       m->smear_lambda, m->layers[0].resid_lambda, m->layers[0].x0_lambda, ch->tokens, ch->row_off,
                       ch->start, ch->max_per_row, Mcap, D, c->cap, c->hist, w.x, w.x0, w.tok_row, w.tok_pos,
                       full_smear, nullptr, DraftMerge{});
  FC_LAUNCH_CHECK();

  Pending pend{};
  auto norm = [&](int rows, int n_out) {
    const int* md = n_out > 0 ? nullptr : Mdev;
    if (dt == FC_BF16)
      hipLaunchKernelGGL(k_rmsnorm<bf16_t>, dim3(rows), dim3(256), 0, s, w.x, (bf16_t*)w.h, D, Mcap, md, ch->row_off,
                         n_out, pend);
    else
      hipLaunchKernelGGL(k_rmsnorm<float>, dim3(rows), dim3(256), 0, s, w.x, (float*)w.h, D, Mcap, md, ch->row_off,
                         n_out, pend);
    pend = Pending{};
  };
  const int backout = m->n_layer / 2;
  for (int l = 0; l < m->n_layer; ++l) {
    const fc_layer& L = m->layers[l];
    if (l > 0 || !embed_norm) {
      norm(Mcap, 0);
      FC_LAUNCH_CHECK();
    }
    Epi e{};
    if (fuse_qkv) {  // the QKV GEMM finishes RoPE / QK-norm / VE gate / KV append itself
      e.mode = EPI_QKV;
      QkvEpi& Q = e.qkv;
      Q.tokens = ch->tokens;
      Q.tok_row = w.tok_row;
      Q.tok_pos = w.tok_pos;
      Q.rcos = m->rope_cos;
      Q.rsin = m->rope_sin;
      Q.rope_len = m->rope_len;
      Q.ve = (const uint16_t*)L.ve;
      Q.ve_gate = L.ve_gate;
      Q.h = (const uint16_t*)w.h;
      Q.D = D;
      Q.H = H;
      Q.G = G;
      Q.B = B;
      Q.cap = c->cap;
      Q.kc = (uint16_t*)c->k + layer_elems * l;
      Q.vc = (uint16_t*)c->v + layer_elems * l;
      Q.q = (uint16_t*)w.q;
      rc = fc_launch_gemm(w.h, L.wqkv, Mcap, Mdev, Mtyp, NQKV, D, dt, e, w.gw, s, nullptr);
      if (rc) return rc;
    } else {
      e.mode = EPI_STORE;
      e.out = w.qkv;
      e.ldo = NQKV;
      rc = fc_launch_gemm(w.h, L.wqkv, Mcap, Mdev, Mtyp, NQKV, D, dt, e, w.gw, s, nullptr);
      if (rc) return rc;
      rc = fc_launch_prologue(w.qkv, w.h, ch->tokens, m, l, c, w.tok_row, w.tok_pos, Mcap, Mdev, w.q, s);
      if (rc) return rc;
    }
    int max_keys = c->cap;
    if (L.window > 0) max_keys = std::min(c->cap, L.window + ch->max_per_row);
    rc = fc_launch_attention(w.q, (const char*)c->k + layer_elems * l * es, (const char*)c->v + layer_elems * l * es,
                             w.y, B, Mcap, ch->max_per_row, typ_per_row, H, G, hd, c->cap, ch->row_off, ch->start,
                             L.window, max_keys, dt, w.part, w.part_bytes, s);
    if (rc) return rc;
    e = Epi{};
    e.mode = EPI_ADD;
    e.out = w.x;
    e.ldo = D;
    int S = 1;
    if (fold) {  // x += attn; h = bf16(x) and per-tile sums of squares for c_fc
      e.xa = (uint16_t*)w.h;
      e.ssq = w.ssq;
      e.ssq_ld = Mcap;
      rc = fc_launch_gemm(w.y, L.wo, Mcap, Mdev, Mtyp, D, H * hd, dt, e, w.gw, s, nullptr);
      if (rc) return rc;
    } else {
      rc = fc_launch_gemm(w.y, L.wo, Mcap, Mdev, Mtyp, D, H * hd, dt, e, w.gw, s, &S);
      if (rc) return rc;
      if (S > 1) {
        pend.S = S;
        pend.mode = EPI_ADD;
        pend.rows = Mcap;
        pend.part = w.gw.part;
      }
      norm(Mcap, 0);
      FC_LAUNCH_CHECK();
    }
    e = Epi{};
    e.mode = EPI_RELU2;
    e.out = w.hid;
    e.ldo = 4 * D;
    e.out_dtype = dt;
    if (fold) {
      e.rms_in = w.ssq;
      e.rms_n = fc_gemm_fold_tiles(Mtyp, D);
      e.ssq_ld = Mcap;
    }
    rc = fc_launch_gemm(w.h, L.wfc, Mcap, Mdev, Mtyp, 4 * D, D, dt, e, w.gw, s, nullptr);
    if (rc) return rc;
    e = Epi{};
    e.mode = EPI_MLPOUT;
    e.out = w.x;
    e.ldo = D;
    e.x0 = w.x0;
    e.xb = w.xb;
    e.capture = l == backout;
    e.last = l == m->n_layer - 1;
    e.lb = m->backout_lambda;
    if (!e.last) {
      e.r = m->layers[l + 1].resid_lambda;
      e.a = m->layers[l + 1].x0_lambda;
    }
    S = 1;
    rc = fc_launch_gemm(w.hid, L.wproj, Mcap, Mdev, Mtyp, D, 4 * D, dt, e, w.gw, s, &S);
    if (rc) return rc;
    if (S > 1) {
      pend.S = S;
      pend.mode = EPI_MLPOUT;
      pend.rows = Mcap;
      pend.part = w.gw.part;
      pend.x0 = w.x0;
      pend.xb = w.xb;
      pend.r = e.r;
      pend.a = e.a;
      pend.lb = e.lb;
      pend.capture = e.capture;
      pend.last = e.last;
    }
  }
  if (ch->n_out > 0) {
    const int Mo = B * ch->n_out;
    norm(Mo, ch->n_out);
    FC_LAUNCH_CHECK();
    Epi e{};
    e.mode = EPI_SOFTCAP;
    e.out = ch->logits;
    e.n_out = ch->n_out;
    e.row_stride = ch->logits_stride;
    e.V = m->vocab;
    // the draft step's vocab pass folded into its logits GEMM where the
    // kernel can take it and the caller's partials buffer holds a VPart per
    // row and column tile
    const int vt = vpf != nullptr && vpf->vp != nullptr ? fc_gemm_vocab_tiles(Mo, m->vocab_pad, D, dt) : 0;
    if (vt > 0 && vt <= vpf->max_tiles && (int64_t)Mo * vt <= vpf->vp_cap) {
      e.vp = vpf->vp;
      e.vp_ld = vt;
      e.vp_T = vpf->T;
      e.vp_draw = vpf->draw;
      e.vp_slot = vpf->slot;
      e.vp_seed = vpf->seed;
      e.vp_round = vpf->round;
    }
    rc = fc_launch_gemm(w.h, m->lm_head, Mo, nullptr, Mo, m->vocab_pad, D, dt, e, w.gw, s, nullptr);
    if (rc) return rc;
    if (e.vp != nullptr) *nch = vt;
  }
  return FC_OK;
}

// QKV projection of one layer with its attention prologue: the fused GEMM
// epilogue (EPI_QKV) where the plan provides one (bf16, head_dim 128, verify
// and prefill row counts), else the GEMM into `work` and k_prologue.
extern "C" int64_t fc_attn_qkv_workspace_bytes(const fc_model* m, int32_t M, int32_t typ_tokens) {
  if (!m || M <= 0 || m->n_head <= 0 || m->n_kv_head <= 0) return -1;
  const int hd = m->head_dim, NQKV = (m->n_head + 2 * m->n_kv_head) * hd;
  if (fc_gemm_fuses_qkv(typ_of(M, typ_tokens), NQKV, m->n_embd, m->dtype, hd)) return 0;
  return fc_align((int64_t)M * NQKV * 4);
}

extern "C" int32_t fc_attn_qkv(const fc_model* m, int32_t layer, const fc_cache* c, const void* h,
                               const int32_t* tokens, const int32_t* tok_row, const int32_t* tok_pos, int32_t M,
                               int32_t typ_tokens, void* q, void* work, int64_t work_bytes, void* stream) {
  int rc = check_model(m);
  if (rc) return rc;
  FC_CHECK_ARG(c && c->k && c->v && c->batch > 0 && c->cap > 0 && c->cap % 32 == 0, "cache");
  FC_CHECK_ARG(h && tokens && tok_row && tok_pos && q, "null pointer");
  FC_CHECK_ARG(layer >= 0 && layer < m->n_layer, "layer out of range");
  FC_CHECK_ARG(M >= 0, "M");
  if (M == 0) return FC_OK;
  hipStream_t s = (hipStream_t)stream;
  const int D = m->n_embd, H = m->n_head, G = m->n_kv_head, hd = m->head_dim;
  const int NQKV = (H + 2 * G) * hd, Mtyp = typ_of(M, typ_tokens);
  const fc_layer& L = m->layers[layer];
  const int64_t need = fc_attn_qkv_workspace_bytes(m, M, typ_tokens);
  FC_CHECK_ARG(need == 0 || (work && work_bytes >= need), "fc_attn_qkv workspace too small");
  Epi e{};
  if (need == 0) {
    e.mode = EPI_QKV;
    QkvEpi& Q = e.qkv;
    Q.tokens = tokens;
    Q.tok_row = tok_row;
    Q.tok_pos = tok_pos;
    Q.rcos = m->rope_cos;
    Q.rsin = m->rope_sin;
    Q.rope_len = m->rope_len;
    Q.ve = (const uint16_t*)L.ve;
    Q.ve_gate = L.ve_gate;
    Q.h = (const uint16_t*)h;
    Q.D = D;
    Q.H = H;
    Q.G = G;
    Q.B = c->batch;
    Q.cap = c->cap;
    const int64_t layer_elems = (int64_t)c->batch * G * c->cap * hd;
    Q.kc = (uint16_t*)c->k + layer_elems * layer;
    Q.vc = (uint16_t*)c->v + layer_elems * layer;
    Q.q = (uint16_t*)q;
    return fc_launch_gemm(h, L.wqkv, M, nullptr, Mtyp, NQKV, D, m->dtype, e, GemmWork{}, s, nullptr);
  }
  e.mode = EPI_STORE;
  e.out = work;
  e.ldo = NQKV;
  rc = fc_launch_gemm(h, L.wqkv, M, nullptr, Mtyp, NQKV, D, m->dtype, e, GemmWork{}, s, nullptr);
  if (rc) return rc;
  return fc_launch_prologue((const float*)work, h, tokens, m, layer, c, tok_row, tok_pos, M, nullptr, q, s);
}

// Streaming read of `bytes` bytes (the measured read ceiling the benchmark
// rates the HBM-bound kernels against): each workgroup streams one
// contiguous share with 16-byte non-temporal loads, four in flight per
// thread, folded with xor into one word per wave so the loads cannot be
// dropped. (A grid-stride order over the whole buffer reads ~10% slower.)
typedef uint32_t rp_u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void k_read_probe(const rp_u32x4* __restrict__ src, int64_t n16,
                                                    uint32_t* __restrict__ out) {
  // workgroup b streams the contiguous range [b per, (b + 1) per) of 16-byte
  // entries, each step 4 KB per load instruction group x 4 in flight
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t b0 = (int64_t)blockIdx.x * per, b1 = min(b0 + per, n16);
  int64_t i = b0 + threadIdx.x;
  rp_u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + 3 * 256 < b1; i += 4 * 256) {
    const rp_u32x4 a = __builtin_nontemporal_load(src + i), b = __builtin_nontemporal_load(src + i + 256);
    const rp_u32x4 c = __builtin_nontemporal_load(src + i + 512);
    const rp_u32x4 d = __builtin_nontemporal_load(src + i + 768);
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < b1; i += 256) acc ^= __builtin_nontemporal_load(src + i);
  uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o, WAVE);
  if ((threadIdx.x & 63) == 0) out[blockIdx.x * 4 + (threadIdx.x >> 6)] = x;
}

extern "C" int32_t fc_read_probe(const void* src, int64_t bytes, uint32_t* out, int32_t workgroups, void* stream) {
  FC_CHECK_ARG(src && out, "null pointer");
  FC_CHECK_ARG(bytes > 0 && bytes % 16 == 0, "bytes must be a positive multiple of 16");
  FC_CHECK_ARG(workgroups > 0 && workgroups <= 65536, "workgroups in [1, 65536]");
  hipLaunchKernelGGL(k_read_probe, dim3(workgroups), dim3(256), 0, (hipStream_t)stream, (const rp_u32x4*)src,
                     bytes / 16, out);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

// Read of L2-resident data (the ceiling against which the GEMMs' L2-to-CU
// traffic is rated): workgroup w reads `per_wg` bytes from the region of XCD
// w % 8 (workgroups are dealt to the eight XCDs round robin, so each XCD's L2
// holds its own region of `region` bytes), starting at offset 64 KB x (w / 8)
// and wrapping. Direct global-to-LDS loads (16 bytes per lane), sixteen 1 KB
// loads in flight per wave, the data landing in a per-wave LDS ring that
// nothing reads (one word of it is folded into `out` at the end).
#define L2P_DEPTH 16
__global__ __launch_bounds__(256) void k_l2_probe(const char* __restrict__ src, int64_t region, int64_t per_wg,
                                                  uint32_t* __restrict__ out) {
  __shared__ uint4 ring[4][L2P_DEPTH][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const char* base = src + (int64_t)(blockIdx.x & 7) * region;
  // each step the workgroup reads 4 KB: wave w the 1 KB at offset 1 KB w
  int64_t off = ((int64_t)(blockIdx.x >> 3) * 65536) % region;
  const int64_t steps = per_wg / 4096;
  for (int64_t it = 0; it < steps; it += L2P_DEPTH) {
#pragma unroll
    for (int u = 0; u < L2P_DEPTH; ++u) {
      __builtin_amdgcn_global_load_lds((const void*)(base + off + wave * 1024 + lane * 16),
                                       (__attribute__((address_space(3))) void*)&ring[wave][u][0], 16, 0, 0);
      off += 4096;
      if (off >= region) off -= region;
      // at most L2P_DEPTH loads of this wave outstanding
      __builtin_amdgcn_s_waitcnt(((L2P_DEPTH - 1) & 15) | (((L2P_DEPTH - 1) >> 4) << 14) | (7 << 4) | (15 << 8));
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const uint4 v = ring[wave][0][lane];
  uint32_t x = v.x ^ v.y ^ v.z ^ v.w;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o, WAVE);
  if (lane == 0) out[blockIdx.x * 4 + wave] = x;
}

extern "C" int32_t fc_l2_read_probe(const void* src, int64_t region_bytes, int64_t bytes, uint32_t* out,
                                    int32_t workgroups, void* stream) {
  FC_CHECK_ARG(src && out, "null pointer");
  FC_CHECK_ARG(region_bytes >= 65536 && region_bytes % 4096 == 0, "region_bytes: a multiple of 4 KB, >= 64 KB");
  FC_CHECK_ARG(workgroups > 0 && workgroups <= 65536, "workgroups in [1, 65536]");
  const int64_t per_wg = bytes / workgroups / (4096 * L2P_DEPTH) * (4096 * L2P_DEPTH);
  FC_CHECK_ARG(per_wg > 0, "bytes must give each workgroup at least 64 KB");
  hipLaunchKernelGGL(k_l2_probe, dim3(workgroups), dim3(256), 0, (hipStream_t)stream, (const char*)src,
                     region_bytes, per_wg, out);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

// The decode attention's load pattern with no compute: workgroup u (4
// waves) walks unit u's `tiles` contiguous 16 KB tiles (a 32-key K block and
// its V block), wave w taking tiles w, w + 4, ...; per tile each wave issues
// sixteen 1 KB non-temporal loads (16 bytes per lane) and waits for them,
// as k_attn_mfma does. The rate the attention can reach with its grid and
// tile walk, whatever its MFMA and softmax work.
__global__ __launch_bounds__(256) void k_walk_probe(const rp_u32x4* __restrict__ src, int tiles,
                                                    uint32_t* __restrict__ out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const char* ub = (const char*)src + (int64_t)blockIdx.x * tiles * 16384;
  rp_u32x4 acc = {0u, 0u, 0u, 0u};
  for (int t = wave; t < tiles; t += 4) {
    const rp_u32x4* p = (const rp_u32x4*)(ub + (int64_t)t * 16384) + lane;
    rp_u32x4 r[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) r[i] = __builtin_nontemporal_load(p + 64 * i);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc ^= r[i];
  }
  out[blockIdx.x * 256 + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

extern "C" int32_t fc_walk_probe(const void* src, int32_t units, int32_t tiles, uint32_t* out, void* stream) {
  FC_CHECK_ARG(src && out, "null pointer");
  FC_CHECK_ARG(units > 0 && units <= 65535 && tiles > 0, "units in [1, 65535], tiles > 0");
  hipLaunchKernelGGL(k_walk_probe, dim3(units), dim3(256), 0, (hipStream_t)stream, (const rp_u32x4*)src, tiles, out);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

// A GEMM's operand walk without its arithmetic: the blocks the K-split,
// LDS-shared and ring kernels read, in their order, timed by the benchmark
// against the GEMMs themselves. Operands in fragment order (1 KB blocks of
// 16 rows x 32 k, [row block][k step]); output tile (mt, nt) of tile_m x
// tile_n and K split s; XCD x takes the grid's tiles [x per_xcd, (x + 1)
// per_xcd), M tile fastest (the M tiles that share a weight slab on one
// XCD). The split's range is cut into 64-deep k chunks (two k steps), as
// the kernels cut it; wave w takes chunks w, w + 4, ... and per chunk loads
// the tile's W blocks then its A blocks (row blocks past the last live one
// clamped, as the kernels do), each block's two k steps back to back (2 KB
// contiguous), 1 KB per load instruction (16 bytes per lane), at most
// GWP_DEPTH in flight, no barrier.
//   REG = false: direct global-to-LDS loads (k_gemm_dma, k_gemm_ring); the
//     wave's word is the XOR over lanes and words of the LDS slots its last
//     min(loads, 16) loads landed in.
//   REG = true: loads into registers, GWP_DEPTH issued then consumed
//     (k_gemm_ks, k_gemm_la's weights); the wave's word is the XOR of every
//     block it loaded.
#define GWP_DEPTH 16
template <bool REG>
__global__ __launch_bounds__(256) void k_gemm_walk_probe(const char* __restrict__ A, const char* __restrict__ W,
                                                         int M, int KS, int mb, int nb, int mtiles, int ntiles,
                                                         int S, int per_xcd, uint32_t* __restrict__ out) {
  __shared__ uint4 ring[REG ? 1 : 4][16][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int t = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if ((int)(blockIdx.x >> 3) >= per_xcd || t >= mtiles * ntiles * S) return;
  const int mt = t % mtiles, rest = t / mtiles, sp = rest % S, nt = rest / S;
  const int C = KS >> 1;  // 64-deep chunks
  const int c0 = (int)((int64_t)sp * C / S), c1 = (int)((int64_t)(sp + 1) * C / S);
  const int last_blk = (M - 1) >> 4;
  const int per_c = 2 * (mb + nb);
  // the wave's loads in order: load j is chunk c0 + wave + 4 (j / per_c);
  // within it, u = j % per_c: block u / 2 (W blocks first), k step 2 c + u % 2
  const int nch = c1 - c0 > wave ? (c1 - c0 - wave + 3) >> 2 : 0;
  const int nload = nch * per_c;
  auto addr = [&](int j) {
    const int c = c0 + wave + 4 * (j / per_c), u = j % per_c, b = u >> 1, ks = 2 * c + (u & 1);
    const int64_t blk = b < nb ? (int64_t)(nt * nb + b) * KS + ks
                               : (int64_t)min(mt * mb + b - nb, last_blk) * KS + ks;
    return (b < nb ? W : A) + blk * 1024 + lane * 16;
  };
  uint32_t x = 0u;
  if constexpr (REG) {
    for (int j0 = 0; j0 < nload; j0 += GWP_DEPTH) {
      uint4 r[GWP_DEPTH];
#pragma unroll
      for (int u = 0; u < GWP_DEPTH; ++u) r[u] = *(const uint4*)addr(min(j0 + u, nload - 1));
#pragma unroll
      for (int u = 0; u < GWP_DEPTH; ++u)
        if (j0 + u < nload) x ^= r[u].x ^ r[u].y ^ r[u].z ^ r[u].w;
    }
  } else {
    for (int j = 0; j < nload; ++j) {
      __builtin_amdgcn_global_load_lds((const void*)addr(j),
                                       (__attribute__((address_space(3))) void*)&ring[wave][j & 15][0], 16, 0, 0);
      __builtin_amdgcn_s_waitcnt(((GWP_DEPTH - 1) & 15) | (((GWP_DEPTH - 1) >> 4) << 14) | (7 << 4) | (15 << 8));
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads have landed in its own slots
    for (int j = 0; j < min(nload, 16); ++j) {
      const uint4 v = ring[wave][j][lane];
      x ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o, WAVE);
  if (lane == 0) out[blockIdx.x * 4 + wave] = x;
}

extern "C" int32_t fc_gemm_walk_probe_words(int32_t M, int32_t N, int32_t tile_m, int32_t tile_n, int32_t splits) {
  if (M <= 0 || N <= 0 || tile_m <= 0 || tile_n <= 0 || splits <= 0) return -1;
  const int64_t tiles = (int64_t)((M + tile_m - 1) / tile_m) * (N / tile_n) * splits;
  return (int32_t)(4 * 8 * ((tiles + 7) / 8));
}

extern "C" int32_t fc_gemm_walk_probe(const void* A, const void* W, int32_t M, int32_t N, int32_t K, int32_t tile_m,
                                      int32_t tile_n, int32_t splits, int32_t reg_loads, uint32_t* out, void* stream) {
  FC_CHECK_ARG(A && W && out, "null pointer");
  FC_CHECK_ARG(M > 0 && N > 0 && K > 0 && K % 64 == 0, "M, N > 0 and K a positive multiple of 64");
  FC_CHECK_ARG(tile_m > 0 && tile_m % 16 == 0 && tile_n > 0 && tile_n % 16 == 0 && N % tile_n == 0,
               "tiles: multiples of 16, tile_n dividing N");
  FC_CHECK_ARG(splits >= 1 && splits <= K / 64, "splits in [1, K / 64]");
  const int mtiles = (M + tile_m - 1) / tile_m, ntiles = N / tile_n;
  const int64_t tiles = (int64_t)mtiles * ntiles * splits;
  FC_CHECK_ARG(tiles <= (1 << 20), "at most 2^20 tiles");
  const int per_xcd = (int)((tiles + 7) / 8);
  if (reg_loads)
    hipLaunchKernelGGL(k_gemm_walk_probe<true>, dim3(8 * per_xcd), dim3(256), 0, (hipStream_t)stream,
                       (const char*)A, (const char*)W, M, K / 32, tile_m / 16, tile_n / 16, mtiles, ntiles, splits,
                       per_xcd, out);
  else
    hipLaunchKernelGGL(k_gemm_walk_probe<false>, dim3(8 * per_xcd), dim3(256), 0, (hipStream_t)stream,
                       (const char*)A, (const char*)W, M, K / 32, tile_m / 16, tile_n / 16, mtiles, ntiles, splits,
                       per_xcd, out);
  FC_LAUNCH_CHECK();
  return FC_OK;
}
