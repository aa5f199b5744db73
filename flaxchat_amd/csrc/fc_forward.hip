// Chunked multi-token forward: embedding + smear, the transformer blocks and
// the softcapped head, on a preallocated KV cache.
//
// One call replaces `_single_step_forward` (flaxchat/engine.py:51-177) for
// every valid slot of every row at once: the draft's 1-token steps, the
// target's (k+1)-token verify chunk and prompt prefill are the same code
// with a different chunk width W. Activations between kernels:
//   x, x0, xb   fp32 residual stream, x0 and the backout capture
//   h           RMS-normed GEMM input (model dtype)
//   qkv         fp32 projections, consumed by the prologue
//   q, y, hid   attention query / output and the ReLU^2 hidden (model dtype)
#include "fc_common.h"
#include "fc_internal.h"

#define EMBED_MAXW 1024

// Embedding + RMSNorm + smear (flaxchat/engine.py:80-94). The smear chain
// x_t = n_t + g_t * x_{t-1} is sequential in t but elementwise in the model
// dimension, so each thread walks the slots for its own columns.
template <typename T>
__global__ __launch_bounds__(256) void k_embed(const T* __restrict__ wte, const float* __restrict__ smear_gate,
                                               float smear_lambda, float r0, float a0,
                                               const int* __restrict__ tokens, const int* __restrict__ start,
                                               const int* __restrict__ nvalid, int W, int D, int cap,
                                               float* __restrict__ hist, float* __restrict__ x,
                                               float* __restrict__ x0) {
  __shared__ float sg[EMBED_MAXW], sinv[EMBED_MAXW];
  const int b = blockIdx.x;
  const int n = nvalid[b], s0 = start[b], off = W - n;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int j = wave; j < n; j += 4) {
    const int tok = tokens[(int64_t)b * W + off + j];
    const T* e = wte + (int64_t)tok * D;
    float ss = 0.f;
    for (int d = lane; d < D; d += 64) {
      const float v = ld<T>(e, d);
      ss += v * v;
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
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float prev = s0 > 0 ? hist[((int64_t)b * cap + s0 - 1) * D + d] : 0.f;
    for (int j = 0; j < off; ++j) {
      const int64_t m = (int64_t)b * W + j;
      x[m * D + d] = 0.f;
      x0[m * D + d] = 0.f;
    }
    for (int j = 0; j < n; ++j) {
      const int tok = tokens[(int64_t)b * W + off + j];
      const float nv = ld<T>(wte, (int64_t)tok * D + d) * sinv[j];
      const float xv = nv + sg[j] * prev;
      const int pos = s0 + j;
      if (pos < cap) hist[((int64_t)b * cap + pos) * D + d] = xv;
      const int64_t m = (int64_t)b * W + off + j;
      x0[m * D + d] = xv;
      x[m * D + d] = r0 * xv + a0 * xv;
      prev = xv;
    }
  }
}

// h = x * rsqrt(mean(x^2) + 1e-6) (flaxchat/gpt.py:44-46). With n_out > 0,
// output row m reads input row (m / n_out) * W + (W - n_out) + m % n_out
// (the head only needs the last n_out slots of each row).
template <typename TO>
__global__ __launch_bounds__(256) void k_rmsnorm(const float* __restrict__ x, TO* __restrict__ h, int D, int W,
                                                 int n_out) {
  __shared__ float red[16];
  const int row = blockIdx.x;
  const int64_t in_row = n_out > 0 ? (int64_t)(row / n_out) * W + (W - n_out) + row % n_out : row;
  const float* xr = x + in_row * D;
  float ss = 0.f;
  for (int d = threadIdx.x; d < D; d += blockDim.x) ss += xr[d] * xr[d];
  ss = block_sum(ss, red);
  const float inv = 1.f / sqrtf(ss / (float)D + 1e-6f);
  TO* hr = h + (int64_t)row * D;
  for (int d = threadIdx.x; d < D; d += blockDim.x) st<TO>(hr, d, xr[d] * inv);
}

struct FwdWork {
  float *x, *x0, *xb, *qkv;
  void *h, *q, *y, *hid, *part;
  int64_t part_bytes, total;
};

static FwdWork carve(const fc_model* m, int B, int W, int max_keys, char* base) {
  const int64_t M = (int64_t)B * W;
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
  w.h = take(M * D * es);
  w.q = take(M * H * hd * es);
  w.y = take(M * H * hd * es);
  w.hid = take(M * 4 * D * es);
  w.part_bytes = fc_attn_part_bytes(B, W, H, G, hd, max_keys);
  w.part = take(w.part_bytes);
  w.total = off;
  return w;
}

extern "C" int64_t fc_forward_workspace_bytes(const fc_model* m, int32_t batch, int32_t W, int32_t n_out) {
  (void)n_out;
  if (!m || batch <= 0 || W <= 0) return -1;
  // attention splits are sized for the largest key range the cache can hold
  return carve(m, batch, W, 1 << 20, nullptr).total;
}

static int check_model(const fc_model* m) {
  FC_CHECK_ARG(m && m->layers && m->wte && m->lm_head, "model pointers");
  FC_CHECK_ARG(m->dtype == FC_F32 || m->dtype == FC_BF16, "dtype");
  FC_CHECK_ARG(m->n_head > 0 && m->n_kv_head > 0 && m->n_head % m->n_kv_head == 0, "heads");
  FC_CHECK_ARG(m->head_dim * m->n_head == m->n_embd, "head_dim * n_head must equal n_embd");
  FC_CHECK_ARG(m->n_embd % 8 == 0 && m->n_embd >= 24, "n_embd must be a multiple of 8 and >= 24");
  FC_CHECK_ARG(m->vocab > 0 && m->vocab <= m->vocab_pad, "vocab");
  return FC_OK;
}

extern "C" int32_t fc_forward(const fc_model* m, const fc_cache* c, const fc_chunk* ch, void* work,
                              int64_t work_bytes, void* stream) {
  int rc = check_model(m);
  if (rc) return rc;
  FC_CHECK_ARG(c && c->k && c->v && c->hist && c->batch > 0 && c->cap > 0 && c->cap % 32 == 0, "cache");
  FC_CHECK_ARG(ch && ch->W > 0 && ch->W <= EMBED_MAXW && ch->tokens && ch->start && ch->nvalid, "chunk");
  FC_CHECK_ARG(ch->n_out >= 0 && ch->n_out <= ch->W, "n_out");
  FC_CHECK_ARG(ch->n_out == 0 || ch->logits, "logits pointer");
  hipStream_t s = (hipStream_t)stream;
  const int B = c->batch, W = ch->W, M = B * W;
  const int D = m->n_embd, H = m->n_head, G = m->n_kv_head, hd = m->head_dim;
  const int NQKV = (H + 2 * G) * hd;
  FwdWork w = carve(m, B, W, 1 << 20, (char*)work);
  FC_CHECK_ARG(work && work_bytes >= w.total, "forward workspace too small");
  const int dt = m->dtype;
  const int64_t layer_elems = (int64_t)B * G * c->cap * hd;
  const int es = dt == FC_BF16 ? 2 : 4;

  if (dt == FC_BF16)
    hipLaunchKernelGGL(k_embed<bf16_t>, dim3(B), dim3(256), 0, s, (const bf16_t*)m->wte, m->smear_gate,
                       m->smear_lambda, m->layers[0].resid_lambda, m->layers[0].x0_lambda, ch->tokens, ch->start,
                       ch->nvalid, W, D, c->cap, c->hist, w.x, w.x0);
  else
    hipLaunchKernelGGL(k_embed<float>, dim3(B), dim3(256), 0, s, (const float*)m->wte, m->smear_gate,
                       m->smear_lambda, m->layers[0].resid_lambda, m->layers[0].x0_lambda, ch->tokens, ch->start,
                       ch->nvalid, W, D, c->cap, c->hist, w.x, w.x0);
  FC_LAUNCH_CHECK();

  auto norm = [&](int rows, int n_out) {
    if (dt == FC_BF16)
      hipLaunchKernelGGL(k_rmsnorm<bf16_t>, dim3(rows), dim3(256), 0, s, w.x, (bf16_t*)w.h, D, W, n_out);
    else
      hipLaunchKernelGGL(k_rmsnorm<float>, dim3(rows), dim3(256), 0, s, w.x, (float*)w.h, D, W, n_out);
  };
  const int backout = m->n_layer / 2;
  for (int l = 0; l < m->n_layer; ++l) {
    const fc_layer& L = m->layers[l];
    norm(M, 0);
    FC_LAUNCH_CHECK();
    Epi e{};
    e.mode = EPI_STORE;
    e.out = w.qkv;
    e.ldo = NQKV;
    rc = fc_launch_gemm(w.h, L.wqkv, M, NQKV, D, dt, e, s);
    if (rc) return rc;
    rc = fc_launch_prologue(w.qkv, w.h, ch->tokens, m, l, c, ch->start, ch->nvalid, B, W, w.q, s);
    if (rc) return rc;
    int max_keys = c->cap;
    if (L.window > 0) max_keys = std::min(c->cap, L.window + W);
    rc = fc_launch_attention(w.q, (const char*)c->k + layer_elems * l * es, (const char*)c->v + layer_elems * l * es,
                             w.y, B, W, H, G, hd, c->cap, ch->start, ch->nvalid, L.window, max_keys, dt, w.part,
                             w.part_bytes, s);
    if (rc) return rc;
    e = Epi{};
    e.mode = EPI_ADD;
    e.out = w.x;
    e.ldo = D;
    rc = fc_launch_gemm(w.y, L.wo, M, D, H * hd, dt, e, s);
    if (rc) return rc;
    norm(M, 0);
    FC_LAUNCH_CHECK();
    e = Epi{};
    e.mode = EPI_RELU2;
    e.out = w.hid;
    e.ldo = 4 * D;
    e.out_dtype = dt;
    rc = fc_launch_gemm(w.h, L.wfc, M, 4 * D, D, dt, e, s);
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
    rc = fc_launch_gemm(w.hid, L.wproj, M, D, 4 * D, dt, e, s);
    if (rc) return rc;
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
    rc = fc_launch_gemm(w.h, m->lm_head, Mo, m->vocab_pad, D, dt, e, s);
    if (rc) return rc;
  }
  return FC_OK;
}
