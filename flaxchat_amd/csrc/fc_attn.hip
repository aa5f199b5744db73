// Per-token attention prologue and split-KV flash-decode attention.
//
// Prologue (flaxchat/engine.py:96-126, flaxchat/gpt.py:65-71): value
// embedding gate on the V heads, RoPE (base 100000) and 1.2 * RMSNorm on
// the Q and K heads, then the K/V append at each valid slot's position.
//
// Attention (flaxchat/engine.py:128-156): for query position p and KV
// group g = h / (H / G), softmax over keys j with j <= p and, for layers
// with a window W > 0, p - j <= W (W + 1 keys, inclusive). The reference
// scores every cached position and masks with -1e9; the masked terms are
// exact zeros in fp32, so reading only the visible keys is the same sum.
//
// bf16 path (head_dim 128): one workgroup per (row, KV group, query block of
// 16 columns, key split). Columns are (token, head-in-group) pairs of the
// row's packed tokens, so a verify chunk's tokens and the GQA heads of a
// group share every K/V tile read. Each wave walks 32-key tiles with two matrix-core products:
//   S^T = K Q^T   (16 keys x 16 columns per MFMA; two MFMAs per tile, with
//                  the key rows interleaved so each lane ends up holding 8
//                  consecutive keys of its column), then online softmax in
//                  registers with wave shuffles,
//   O^T += V^T P^T (P taken straight from registers as the B operand; V^T
//                  read from the 32-key blocked-transposed V cache as one
//                  16-byte load per lane).
// The four waves merge in LDS; splits merge in k_attn_combine.
// Prefill-width chunks (>= 128 query columns per row) take k_attn_pf: 128
// columns per workgroup on the 32x32x16 MFMA, K/V tiles shared through LDS.
// fp32 path (parity mode, or head_dim != 128): one workgroup per query with
// the reference's operation order (scores, max, exp, normalise, weighted sum).
#include "fc_common.h"
#include "fc_internal.h"
#include <mutex>
#include <string>

// K/V cache loads are streamed once per call: non-temporal loads keep them
// from displacing reusable lines in the caches (measured ~8% faster at cfg4)
#ifndef FC_ATTN_NT
#define FC_ATTN_NT 1
#endif
#if FC_ATTN_NT
typedef uint32_t kv_u32x4 __attribute__((ext_vector_type(4)));
#define KV_LD(p) __builtin_bit_cast(uint4, __builtin_nontemporal_load((const kv_u32x4*)(p)))
#else
#define KV_LD(p) (*(p))
#endif

// ---------------------------------------------------------------------------
// Prologue: one wave per (packed token m, head slot hh in [0, H + 2G)).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_prologue(const float* __restrict__ qkv, const T* __restrict__ h,
                                                  const int* __restrict__ tokens, const float* __restrict__ rcos,
                                                  const float* __restrict__ rsin, int rope_len,
                                                  const T* __restrict__ ve, const float* __restrict__ ve_gate,
                                                  int D, T* __restrict__ kc, T* __restrict__ vc, int B, int Mcap,
                                                  const int* __restrict__ Mdev, int H, int G, int hd, int cap,
                                                  const int* __restrict__ tok_row, const int* __restrict__ tok_pos,
                                                  T* __restrict__ q, int kblk) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int NH = H + 2 * G;
  const int64_t item = (int64_t)blockIdx.x * 4 + wave;
  if (item >= (int64_t)Mcap * NH) return;
  const int m = (int)(item / NH), hh = (int)(item % NH);
  const int half = hd >> 1;
  const bool act = lane < half;
  const bool vhead = hh >= H + G;
  // every load that needs neither the token's row nor its position (the
  // device total included: a launch covers the chunk's capacity, and the
  // loads of a token past the total stay inside it) is issued before any of
  // them is waited for; tokens past the total then exit, and the rotary table
  // and the value-embedding row follow as one second batch
  const int mdev = Mdev != nullptr ? *Mdev : Mcap;
  const int b = tok_row[m], pos = tok_pos[m];
  const float* row = qkv + ((int64_t)m * NH + hh) * hd;
  float x1 = act ? row[lane] : 0.f, x2 = act ? row[lane + half] : 0.f;
  int tok = 0;
  float part = 0.f;
  if (vhead && ve != nullptr) {
    tok = tokens[m];
    part = lane < 12 ? ld<T>(h, act_idx<T>(m, lane, D)) * ve_gate[(hh - H - G) * 12 + lane] : 0.f;
  }
  if (m >= mdev) return;
  if ((unsigned)b >= (unsigned)B) return;
  if (!vhead) {
    const int pc = min(max(pos, 0), rope_len - 1);
    const float c = act ? rcos[(int64_t)pc * half + lane] : 0.f;
    const float s = act ? rsin[(int64_t)pc * half + lane] : 0.f;
    float y1 = x1 * c + x2 * s;
    float y2 = x1 * (-s) + x2 * c;
    const float ss = wave_sum(y1 * y1 + y2 * y2);
    const float inv = 1.f / sqrtf(ss / (float)hd + 1e-6f);
    y1 = y1 * inv * 1.2f;
    y2 = y2 * inv * 1.2f;
    if (hh < H) {
      if (act) {
        T* qo = q + ((int64_t)m * H + hh) * hd;
        st<T>(qo, lane, y1);
        st<T>(qo, lane + half, y2);
      }
    } else if (act && pos >= 0 && pos < cap) {
      const int g = hh - H;
      T* kg = kc + ((int64_t)b * G + g) * cap * hd;
      if (kblk) {
        st<T>(kg, kblk_idx(pos, lane), y1);
        st<T>(kg, kblk_idx(pos, lane + half), y2);
      } else {
        st<T>(kg, (int64_t)pos * hd + lane, y1);
        st<T>(kg, (int64_t)pos * hd + lane + half, y2);
      }
    }
  } else {
    const int g = hh - H - G;
    if (ve != nullptr) {
      float v1 = 0.f, v2 = 0.f;
      if (act) {
        const T* vr = ve + ((int64_t)tok * G + g) * hd;
        v1 = ld<T>(vr, lane);
        v2 = ld<T>(vr, lane + half);
      }
      const float z = wave_sum(part);
      const float gate = 3.f * (1.f / (1.f + expf(-z)));
      x1 = x1 + gate * v1;
      x2 = x2 + gate * v2;
    }
    if (act && pos >= 0 && pos < cap) {
      T* vb = vc + ((((int64_t)b * G + g) * (cap / 32) + pos / 32) * hd) * 32;
      st<T>(vb, (int64_t)lane * 32 + (pos & 31), x1);
      st<T>(vb, (int64_t)(lane + half) * 32 + (pos & 31), x2);
    }
  }
}

int fc_launch_prologue(const float* qkv, const void* h, const int* tokens, const fc_model* m, int layer,
                       const fc_cache* c, const int* tok_row, const int* tok_pos, int Mcap, const int* Mdev, void* q,
                       hipStream_t s) {
  const fc_layer& L = m->layers[layer];
  const int H = m->n_head, G = m->n_kv_head, hd = m->head_dim;
  FC_CHECK_ARG(hd <= 128 && hd % 2 == 0, "head_dim must be even and <= 128");
  const int64_t layer_elems = (int64_t)c->batch * G * c->cap * hd;
  const int64_t items = (int64_t)Mcap * (H + 2 * G);
  const dim3 grid((unsigned)((items + 3) / 4));
  if (m->dtype == FC_BF16) {
    bf16_t* kc = (bf16_t*)c->k + layer_elems * layer;
    bf16_t* vc = (bf16_t*)c->v + layer_elems * layer;
    hipLaunchKernelGGL(k_prologue<bf16_t>, grid, dim3(256), 0, s, qkv, (const bf16_t*)h, tokens, m->rope_cos,
                       m->rope_sin, m->rope_len, (const bf16_t*)L.ve, L.ve_gate, m->n_embd, kc, vc, c->batch, Mcap, Mdev, H, G,
                       hd, c->cap, tok_row, tok_pos, (bf16_t*)q, hd == 128 ? 1 : 0);
  } else {
    float* kc = (float*)c->k + layer_elems * layer;
    float* vc = (float*)c->v + layer_elems * layer;
    hipLaunchKernelGGL(k_prologue<float>, grid, dim3(256), 0, s, qkv, (const float*)h, tokens, m->rope_cos,
                       m->rope_sin, m->rope_len, (const float*)L.ve, L.ve_gate, m->n_embd, kc, vc, c->batch, Mcap, Mdev, H, G,
                       hd, c->cap, tok_row, tok_pos, (float*)q, 0);
  }
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int32_t fc_attn_prologue(const fc_model* m, int32_t layer, const fc_cache* c, const float* qkv,
                                    const void* h, const int32_t* tokens, const int32_t* tok_row,
                                    const int32_t* tok_pos, int32_t M, void* q, void* stream) {
  FC_CHECK_ARG(m && c && qkv && h && tokens && tok_row && tok_pos && q, "null pointer");
  FC_CHECK_ARG(layer >= 0 && layer < m->n_layer && m->layers != nullptr, "layer out of range");
  FC_CHECK_ARG(m->dtype == FC_F32 || m->dtype == FC_BF16, "dtype");
  FC_CHECK_ARG(m->n_head > 0 && m->n_kv_head > 0 && m->n_head % m->n_kv_head == 0, "head counts");
  FC_CHECK_ARG(c->k && c->v && c->batch > 0 && c->cap > 0 && c->cap % 32 == 0, "cache");
  FC_CHECK_ARG(M >= 0, "M");
  if (M == 0) return FC_OK;
  return fc_launch_prologue(qkv, h, tokens, m, layer, c, tok_row, tok_pos, M, nullptr, q, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// bf16 MFMA split-KV attention (head_dim 128)
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mfma16a(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                  0, 0);
}
__device__ __forceinline__ uint32_t pack2bf(float lo, float hi) {
  return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}

// One 32-key tile of one wave: scores S^T = K Q^T, online softmax update,
// O^T += V^T P^T (see the kernel comment).
__device__ __forceinline__ void attn_tile(const uint4 (&kf)[2][4], const uint4 (&vf)[8], const uint4 (&qf)[4],
                                          int kb, int g4, bool cvalid, int kbeg, int kend, int lo_c, int pos_c,
                                          float scale_log2, float& m_run, float& l_run, f32x4 (&O)[8]) {
  f32x4 sc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int cc = 0; cc < 2; ++cc)
#pragma unroll
    for (int s = 0; s < 4; ++s) sc[cc] = mfma16a(kf[cc][s], qf[s], sc[cc]);
  float p[8];
  float mt = -INFINITY;
#pragma unroll
  for (int cc = 0; cc < 2; ++cc)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int jj = i + 4 * cc;
      const int key = kb + 8 * g4 + jj;
      const bool ok = cvalid && key >= kbeg && key < kend && key >= lo_c && key <= pos_c;
      p[jj] = ok ? sc[cc][i] * scale_log2 : -INFINITY;
      mt = fmaxf(mt, p[jj]);
    }
  mt = fmaxf(mt, __shfl_xor(mt, 16, WAVE));
  mt = fmaxf(mt, __shfl_xor(mt, 32, WAVE));
  const float m_new = fmaxf(m_run, mt);
  float alpha = 1.f, psum = 0.f;
  if (m_new == -INFINITY) {
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) p[jj] = 0.f;
  } else {
    alpha = exp2f(m_run - m_new);
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      p[jj] = exp2f(p[jj] - m_new);
      psum += p[jj];
    }
  }
  l_run = l_run * alpha + psum;
  m_run = m_new;
  uint4 pf;
  pf.x = pack2bf(p[0], p[1]);
  pf.y = pack2bf(p[2], p[3]);
  pf.z = pack2bf(p[4], p[5]);
  pf.w = pack2bf(p[6], p[7]);
#pragma unroll
  for (int db = 0; db < 8; ++db) {
    O[db] *= alpha;
    O[db] = mfma16a(vf[db], pf, O[db]);
  }
}

// grid (key split, row x KV group, query block): the query block is the
// slowest dimension, so blocks with no query (a row's second block is
// usually empty) are dispatched last and exit at once.
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_attn_mfma(const bf16_t* __restrict__ q, const bf16_t* __restrict__ kc,
                                                       const bf16_t* __restrict__ vc, float* __restrict__ part_o,
                                                       float* __restrict__ part_ml, bf16_t* __restrict__ y, int H,
                                                       int G, int cap, const int* __restrict__ row_off,
                                                       const int* __restrict__ start, int max_per_row, int Mcap,
                                                       int window, int split_keys, int nsplit, int nqblk,
                                                       float scale_log2) {
  constexpr int HD = 128;
  const int split = blockIdx.x, bg = blockIdx.y, qb = blockIdx.z;
  const int b = bg / G, g = bg - b * G, rep = H / G;
  const RowSpan sp = row_span(row_off, b, max_per_row, Mcap);
  const int base = sp.base, n = sp.n, s0 = start[b];
  const int ncol = n * rep;
  if (qb * 16 >= ncol) return;  // no query of this row in the block: combine reads nothing here
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, g4 = lane >> 4;
  const int64_t pidx = ((int64_t)bg * nqblk + qb) * nsplit + split;

  // key range of the whole query block
  const int f = qb * 16, lcol = min(qb * 16 + 15, ncol - 1);
  int kbeg = 0, kend = 0;
  {
    const int pf = s0 + f / rep, pl = s0 + lcol / rep;
    const int klo = window > 0 ? max(0, pf - window) : 0;
    const int khi = min(pl + 1, cap);
    kbeg = klo + split * split_keys;
    kend = min(khi, kbeg + split_keys);
  }
  if (kbeg >= kend) {  // only with several splits: a query always sees itself
    if (threadIdx.x < 16) {
      part_ml[(pidx * 16 + threadIdx.x) * 2 + 0] = -INFINITY;
      part_ml[(pidx * 16 + threadIdx.x) * 2 + 1] = 0.f;
    }
    return;
  }
  // this lane's query column
  const int col = qb * 16 + c;
  const int j = col / rep, head = g * rep + (col - j * rep);
  const bool cvalid = col < ncol;
  const int pos_c = s0 + j;
  const int lo_c = window > 0 ? max(0, pos_c - window) : 0;

  const uint4 zero = {0u, 0u, 0u, 0u};
  uint4 qf[4];
  {
    const bf16_t* qr = q + ((int64_t)(base + (cvalid ? j : 0)) * H + head) * HD + 8 * g4;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = cvalid ? *(const uint4*)(qr + 32 * s) : zero;
  }
  const bf16_t* kbase = kc + (int64_t)bg * cap * HD;
  const bf16_t* vbase = vc + (int64_t)bg * (cap / 32) * HD * 32;
  const int r = c;

  float m_run = -INFINITY, l_run = 0.f;
  f32x4 O[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) O[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // K blocks of 32 keys in fragment order: load (cc, s) of a tile is 1 KB
  // contiguous; V blocks are [128 dims][32 keys], one 1 KB load per db
  const int t0 = kbeg & ~31;
  const int ntiles = (kend - t0 + 31) >> 5;
#define ATT_LOAD(kf, vf, kb_)                                                                      \
  {                                                                                                \
    const bf16_t* kt = kbase + (int64_t)((kb_) >> 5) * 32 * HD + lane * 8;                         \
    _Pragma("unroll") for (int cc = 0; cc < 2; ++cc)                                               \
      _Pragma("unroll") for (int s = 0; s < 4; ++s) kf[cc][s] = KV_LD((const uint4*)(kt + (s * 2 + cc) * 512)); \
    const bf16_t* vt = vbase + (int64_t)((kb_) >> 5) * HD * 32 + r * 32 + 8 * g4;                  \
    _Pragma("unroll") for (int db = 0; db < 8; ++db) vf[db] = KV_LD((const uint4*)(vt + db * 16 * 32));  \
  }
  for (int t = wave; t < ntiles; t += NW) {
    const int kb = t0 + 32 * t;
    uint4 kf[2][4], vf[8];
    ATT_LOAD(kf, vf, kb);
    attn_tile(kf, vf, qf, kb, g4, cvalid, kbeg, kend, lo_c, pos_c, scale_log2, m_run, l_run, O);
  }
#undef ATT_LOAD
  // merge the NW waves in LDS; thread t < 256 then owns column t / 16 and
  // dims 8 (t % 16) .. +7. A single key split writes y directly (normalised,
  // in the c_proj operand layout); otherwise the unnormalised partial and its
  // (max, sum) go to k_attn_combine.
  float l_tot = l_run + __shfl_xor(l_run, 16, WAVE);
  l_tot = l_tot + __shfl_xor(l_tot, 32, WAVE);
  __shared__ float sm[NW][16], sl[NW][16];
  __shared__ float so[NW][16][HD + 4];
  if (g4 == 0) {
    sm[wave][c] = m_run;
    sl[wave][c] = l_tot;
  }
#pragma unroll
  for (int db = 0; db < 8; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) so[wave][c][16 * db + 4 * g4 + i] = O[db][i];
  __syncthreads();
  if (threadIdx.x >= 256) return;
  const int qc = threadIdx.x >> 4, d0 = (threadIdx.x & 15) * 8;
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < NW; ++w) M = fmaxf(M, sm[w][qc]);
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float L = 0.f;
  if (M != -INFINITY) {
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float a = exp2f(sm[w][qc] - M);
      L += a * sl[w][qc];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] += a * so[w][qc][d0 + i];
    }
  }
  if (nsplit == 1) {
    const int colq = qb * 16 + qc;
    if (colq >= ncol) return;
    const int jq = colq / rep, hq = g * rep + (colq - jq * rep);
    const float inv = L > 0.f ? 1.f / L : 0.f;
    uint4 pk;
    pk.x = pack2bf(o[0] * inv, o[1] * inv);
    pk.y = pack2bf(o[2] * inv, o[3] * inv);
    pk.z = pack2bf(o[4] * inv, o[5] * inv);
    pk.w = pack2bf(o[6] * inv, o[7] * inv);
    *(uint4*)(y + frag_idx(base + jq, hq * HD + d0, H * HD)) = pk;
    return;
  }
  float4* po = (float4*)(part_o + (pidx * 16 + qc) * HD + d0);
  po[0] = make_float4(o[0], o[1], o[2], o[3]);
  po[1] = make_float4(o[4], o[5], o[6], o[7]);
  if (d0 == 0) {
    part_ml[(pidx * 16 + qc) * 2 + 0] = M;
    part_ml[(pidx * 16 + qc) * 2 + 1] = L;
  }
}

// The same for QB query blocks per workgroup (GQA verify chunks: tokens x
// heads-per-group > 16 columns): each wave applies every K/V tile it loads
// to all QB blocks, so the key range is read once per QB blocks instead of
// once per block; the waves are merged block by block. grid (key split,
// row x KV group, group of QB query blocks).
template <int NW, int QB>
__global__ __launch_bounds__(64 * NW, 2) void k_attn_mfma_qb(const bf16_t* __restrict__ q, const bf16_t* __restrict__ kc,
                                                       const bf16_t* __restrict__ vc, float* __restrict__ part_o,
                                                       float* __restrict__ part_ml, bf16_t* __restrict__ y, int H,
                                                       int G, int cap, const int* __restrict__ row_off,
                                                       const int* __restrict__ start, int max_per_row, int Mcap,
                                                       int window, int split_keys, int nsplit, int nqblk,
                                                       float scale_log2) {
  constexpr int HD = 128;
  const int split = blockIdx.x, bg = blockIdx.y, qb0 = blockIdx.z * QB;
  const int b = bg / G, g = bg - b * G, rep = H / G;
  const RowSpan sp = row_span(row_off, b, max_per_row, Mcap);
  const int base = sp.base, n = sp.n, s0 = start[b];
  const int ncol = n * rep;
  if (qb0 * 16 >= ncol) return;  // no query of this row in the group: combine reads nothing here
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, g4 = lane >> 4;
  const int nblk = min(QB, (ncol - qb0 * 16 + 15) / 16);  // blocks of the group holding a query

  // key range of the whole group of query blocks
  const int f = qb0 * 16, lcol = min(qb0 * 16 + 16 * QB - 1, ncol - 1);
  int kbeg = 0, kend = 0;
  {
    const int pf = s0 + f / rep, pl = s0 + lcol / rep;
    const int klo = window > 0 ? max(0, pf - window) : 0;
    const int khi = min(pl + 1, cap);
    kbeg = klo + split * split_keys;
    kend = min(khi, kbeg + split_keys);
  }
  if (kbeg >= kend) {  // only with several splits: a query always sees itself
    if (threadIdx.x < 16) {
      for (int u = 0; u < nblk; ++u) {
        const int64_t pidx = ((int64_t)bg * nqblk + qb0 + u) * nsplit + split;
        part_ml[(pidx * 16 + threadIdx.x) * 2 + 0] = -INFINITY;
        part_ml[(pidx * 16 + threadIdx.x) * 2 + 1] = 0.f;
      }
    }
    return;
  }
  // this lane's query column in each block
  bool cvalid[QB];
  int pos_c[QB], lo_c[QB];
  uint4 qf[QB][4];
#pragma unroll
  for (int u = 0; u < QB; ++u) {
    const int col = (qb0 + u) * 16 + c;
    const int j = col / rep, head = g * rep + (col - j * rep);
    cvalid[u] = col < ncol;
    pos_c[u] = s0 + j;
    lo_c[u] = window > 0 ? max(0, pos_c[u] - window) : 0;
    const bf16_t* qr = q + ((int64_t)(base + (cvalid[u] ? j : 0)) * H + (cvalid[u] ? head : 0)) * HD + 8 * g4;
    // load from the (always valid, clamped) address, then mask the value: a
    // select between the load and `zero` becomes a select of pointers, one of
    // them to a private copy of `zero`, and the loads turn into flat loads
    const uint32_t keep = cvalid[u] ? 0xffffffffu : 0u;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint4 v = *(const uint4*)(qr + 32 * s);
      qf[u][s] = uint4{v.x & keep, v.y & keep, v.z & keep, v.w & keep};
    }
  }
  const bf16_t* kbase = kc + (int64_t)bg * cap * HD;
  const bf16_t* vbase = vc + (int64_t)bg * (cap / 32) * HD * 32;
  const int r = c;

  float m_run[QB], l_run[QB];
  f32x4 O[QB][8];
#pragma unroll
  for (int u = 0; u < QB; ++u) {
    m_run[u] = -INFINITY;
    l_run[u] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) O[u][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // K blocks of 32 keys in fragment order: load (cc, s) of a tile is 1 KB
  // contiguous; V blocks are [128 dims][32 keys], one 1 KB load per db
  const int t0 = kbeg & ~31;
  const int ntiles = (kend - t0 + 31) >> 5;
  for (int t = wave; t < ntiles; t += NW) {
    const int kb = t0 + 32 * t;
    uint4 kf[2][4], vf[8];
    const bf16_t* kt = kbase + (int64_t)(kb >> 5) * 32 * HD + lane * 8;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
      for (int s = 0; s < 4; ++s) kf[cc][s] = KV_LD((const uint4*)(kt + (s * 2 + cc) * 512));
    const bf16_t* vt = vbase + (int64_t)(kb >> 5) * HD * 32 + r * 32 + 8 * g4;
#pragma unroll
    for (int db = 0; db < 8; ++db) vf[db] = KV_LD((const uint4*)(vt + db * 16 * 32));
#pragma unroll
    for (int u = 0; u < QB; ++u)
      if (u < nblk)
        attn_tile(kf, vf, qf[u], kb, g4, cvalid[u], kbeg, kend, lo_c[u], pos_c[u], scale_log2, m_run[u], l_run[u],
                  O[u]);
  }
  // merge the NW waves in LDS, block by block; thread t < 256 then owns
  // column t / 16 and dims 8 (t % 16) .. +7. A single key split writes y
  // directly (normalised, in the c_proj operand layout); otherwise the
  // unnormalised partial and its (max, sum) go to k_attn_combine.
  __shared__ float sm[NW][16], sl[NW][16];
  __shared__ float so[NW][16][HD + 4];
  // (a guard instead of a break keeps the loop unrolled, so m_run / l_run / O
  // stay in registers: a runtime index would put them in scratch memory)
#pragma unroll
  for (int u = 0; u < QB; ++u) {
    if (u < nblk) {  // uniform over the workgroup
      const int qb = qb0 + u;
      const int64_t pidx = ((int64_t)bg * nqblk + qb) * nsplit + split;
      float l_tot = l_run[u] + __shfl_xor(l_run[u], 16, WAVE);
      l_tot = l_tot + __shfl_xor(l_tot, 32, WAVE);
      if (u > 0) __syncthreads();  // the previous block's readers are done with the LDS
      if (g4 == 0) {
        sm[wave][c] = m_run[u];
        sl[wave][c] = l_tot;
      }
  #pragma unroll
      for (int db = 0; db < 8; ++db)
  #pragma unroll
        for (int i = 0; i < 4; ++i) so[wave][c][16 * db + 4 * g4 + i] = O[u][db][i];
      __syncthreads();
      if (threadIdx.x < 256) {
        const int qc = threadIdx.x >> 4, d0 = (threadIdx.x & 15) * 8;
        float M = -INFINITY;
  #pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, sm[w][qc]);
        float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        float L = 0.f;
        if (M != -INFINITY) {
  #pragma unroll
          for (int w = 0; w < NW; ++w) {
            const float a = exp2f(sm[w][qc] - M);
            L += a * sl[w][qc];
  #pragma unroll
            for (int i = 0; i < 8; ++i) o[i] += a * so[w][qc][d0 + i];
          }
        }
        const int colq = qb * 16 + qc;
        if (nsplit == 1) {
          if (colq < ncol) {
            const int jq = colq / rep, hq = g * rep + (colq - jq * rep);
            const float inv = L > 0.f ? 1.f / L : 0.f;
            uint4 pk;
            pk.x = pack2bf(o[0] * inv, o[1] * inv);
            pk.y = pack2bf(o[2] * inv, o[3] * inv);
            pk.z = pack2bf(o[4] * inv, o[5] * inv);
            pk.w = pack2bf(o[6] * inv, o[7] * inv);
            *(uint4*)(y + frag_idx(base + jq, hq * HD + d0, H * HD)) = pk;
          }
        } else {
          float4* po = (float4*)(part_o + (pidx * 16 + qc) * HD + d0);
          po[0] = make_float4(o[0], o[1], o[2], o[3]);
          po[1] = make_float4(o[4], o[5], o[6], o[7]);
          if (d0 == 0) {
            part_ml[(pidx * 16 + qc) * 2 + 0] = M;
            part_ml[(pidx * 16 + qc) * 2 + 1] = L;
          }
        }
      }
    }
  }
}

// Prefill attention on the 32x32x16 MFMA. A workgroup owns 128 query
// columns of one (row, KV group), 32 per wave. The 32-key K / V tiles of the
// group's key range go through a 3-stage LDS ring by direct loads (each wave
// 4 of a tile's 16 blocks of 1 KB), so a tile is read once per 128 columns.
// Per tile a wave computes S^T = K Q^T (32 keys x its 32 columns; lane l
// holds column l % 32 and 16 of the keys), the online softmax in registers
// (one swap with lane l ^ 32 per max), then O^T += V^T P^T (4 x 32 dims); the
// P operand of a 16-key half takes 4 keys from the lane and 4 from lane
// l ^ 32. Both K and V are read from LDS in their cache layouts with
// lane-dependent addresses. Waves skip the tiles outside their own key range
// but take part in every load and barrier.
struct PfStage {
  uint4 k[8][64];  // one 32-key block of the K cache (8 KB)
  uint4 v[512];    // one 32-key block of the V cache: [128 dims][32 keys] (8 KB)
};
__global__ __launch_bounds__(256, 2) void k_attn_pf(const bf16_t* __restrict__ q, const bf16_t* __restrict__ kc,
                                                 const bf16_t* __restrict__ vc, bf16_t* __restrict__ y, int H, int G,
                                                 int cap, const int* __restrict__ row_off,
                                                 const int* __restrict__ start, int max_per_row, int Mcap,
                                                 int window, float scale_log2) {
  constexpr int HD = 128;
  __shared__ PfStage st0, st1, st2;
  const int bg = blockIdx.y, b = bg / G, g = bg - b * G, rep = H / G;
  const RowSpan sp = row_span(row_off, b, max_per_row, Mcap);
  const int base = sp.base, n = sp.n, s0 = start[b];
  const int ncol = n * rep;
  const int c0 = blockIdx.x * 128;
  if (c0 >= ncol) return;  // the whole workgroup
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hl = lane >> 5;
  // the workgroup's key range
  const int lcol = min(c0 + 127, ncol - 1);
  const int kbeg = window > 0 ? max(0, s0 + c0 / rep - window) : 0;
  const int kend = min(s0 + lcol / rep + 1, cap);
  const int t0 = kbeg & ~31;
  const int ntiles = (kend - t0 + 31) >> 5;
  // this wave's columns and key range
  const int wc0 = c0 + 32 * wave;
  const bool wact = wc0 < ncol;
  const int w_hi = wact ? s0 + min(wc0 + 31, ncol - 1) / rep : -1;
  const int w_lo = window > 0 ? max(0, s0 + wc0 / rep - window) : 0;
  // tiles inside [w_full_lo, w_full_hi] are visible to every column of the wave (no masks)
  const bool wfull = wc0 + 31 < ncol;
  const int w_full_hi = s0 + wc0 / rep;  // the first column's position
  const int w_full_lo = window > 0 ? max(0, s0 + (wc0 + 31) / rep - window) : 0;
  // this lane's column (query)
  const int col = wc0 + (lane & 31);
  const bool cvalid = col < ncol;
  const int j = cvalid ? col / rep : 0;
  const int head = g * rep + (cvalid ? col - (col / rep) * rep : 0);
  const int pos_c = s0 + j;
  const int lo_c = window > 0 ? max(0, pos_c - window) : 0;
  v4u qf[8];  // dims 16 h + 8 hl .. +7 of this lane's query
  {
    const bf16_t* qr = q + ((int64_t)(base + j) * H + head) * HD + 8 * hl;
#pragma unroll
    for (int h = 0; h < 8; ++h) qf[h] = cvalid ? *(const v4u*)(qr + 16 * h) : v4u{0u, 0u, 0u, 0u};
  }
  // LDS slots this lane reads: K (block, slot) per 16-dim slice h; V uint4 index per (dims block, key half)
  const int kk = lane & 31;
  const int kcc = (kk >> 2) & 1, kr = ((kk >> 3) << 2) | (kk & 3);
  const bf16_t* kbase = kc + (int64_t)bg * cap * HD;
  const bf16_t* vbase = vc + (int64_t)bg * (cap / 32) * HD * 32;
  f32x16 O[4];
#pragma unroll
  for (int dd = 0; dd < 4; ++dd)
#pragma unroll
    for (int x = 0; x < 16; ++x) O[dd][x] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
#define PF_ISSUE(S, t_)                                                                                    \
  {                                                                                                        \
    const int kb_ = t0 + 32 * min((t_), ntiles - 1); /* past the end: harmless re-reads */                 \
    const bf16_t* kt = kbase + (int64_t)(kb_ >> 5) * 32 * HD + lane * 8;                                   \
    const bf16_t* vt = vbase + (int64_t)(kb_ >> 5) * HD * 32 + lane * 8;                                   \
    _Pragma("unroll") for (int u = 0; u < 2; ++u) {                                                        \
      __builtin_amdgcn_global_load_lds((const void*)(kt + (2 * wave + u) * 512),                          \
                                       (__attribute__((address_space(3))) void*)&S.k[2 * wave + u][0], 16, 0, 0); \
      __builtin_amdgcn_global_load_lds((const void*)(vt + (2 * wave + u) * 512),                          \
                                       (__attribute__((address_space(3))) void*)&S.v[64 * (2 * wave + u)], 16, 0, 0); \
    }                                                                                                      \
  }
#define PF_SYNC()                                                                                          \
  {                                                                                                        \
    __builtin_amdgcn_sched_barrier(0);                                                                     \
    __builtin_amdgcn_s_waitcnt((4 & 15) | (7 << 4) | (0 << 8)); /* vmcnt(4): the next tile may be in flight */ \
    __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                               \
    __builtin_amdgcn_sched_barrier(0);                                                                     \
    __builtin_amdgcn_s_barrier();                                                                          \
    __builtin_amdgcn_sched_barrier(0);                                                                     \
    __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                               \
  }
#define PF_TILE(S, t_)                                                                                     \
  {                                                                                                        \
    const int kb = t0 + 32 * (t_);                                                                         \
    if (wact && kb <= w_hi && kb + 31 >= w_lo) {                                                           \
      f32x16 sa, sb;                                                                                       \
      _Pragma("unroll") for (int x = 0; x < 16; ++x) { sa[x] = 0.f; sb[x] = 0.f; }                       \
      _Pragma("unroll") for (int h = 0; h < 8; ++h) {                                                      \
        const int gq = (2 * h + hl) & 3;                                                                   \
        const v4u kf = __builtin_bit_cast(v4u, S.k[2 * (h >> 1) + kcc][kr + 16 * gq]);                    \
        if (h & 1) sb = mfma32(kf, qf[h], sb);                                                             \
        else sa = mfma32(kf, qf[h], sa);                                                                   \
      }                                                                                                    \
      float pv[16];                                                                                        \
      float mt = -INFINITY;                                                                                \
      if (wfull && kb >= w_full_lo && kb + 31 <= w_full_hi) {                                              \
        _Pragma("unroll") for (int i = 0; i < 16; ++i) {                                                   \
          pv[i] = (sa[i] + sb[i]) * scale_log2;                                                            \
          mt = fmaxf(mt, pv[i]);                                                                           \
        }                                                                                                  \
      } else {                                                                                             \
        _Pragma("unroll") for (int i = 0; i < 16; ++i) {                                                   \
          const int key = kb + 8 * (i >> 2) + 4 * hl + (i & 3);                                            \
          const bool ok = cvalid && key >= lo_c && key <= pos_c;                                           \
          pv[i] = ok ? (sa[i] + sb[i]) * scale_log2 : -INFINITY;                                           \
          mt = fmaxf(mt, pv[i]);                                                                           \
        }                                                                                                  \
      }                                                                                                    \
      mt = fmaxf(mt, __shfl_xor(mt, 32, WAVE));                                                            \
      const float m_new = fmaxf(m_run, mt);                                                                \
      float alpha = 1.f, psum = 0.f;                                                                       \
      if (m_new == -INFINITY) {                                                                            \
        _Pragma("unroll") for (int i = 0; i < 16; ++i) pv[i] = 0.f;                                        \
      } else {                                                                                             \
        alpha = __builtin_amdgcn_exp2f(m_run - m_new);                                                     \
        _Pragma("unroll") for (int i = 0; i < 16; ++i) {                                                   \
          pv[i] = __builtin_amdgcn_exp2f(pv[i] - m_new);                                                   \
          psum += pv[i];                                                                                   \
        }                                                                                                  \
      }                                                                                                    \
      l_run = l_run * alpha + psum;                                                                        \
      m_run = m_new;                                                                                       \
      uint2 pk[4];                                                                                         \
      _Pragma("unroll") for (int g4 = 0; g4 < 4; ++g4)                                                     \
        pk[g4] = uint2{pack2bf(pv[4 * g4], pv[4 * g4 + 1]), pack2bf(pv[4 * g4 + 2], pv[4 * g4 + 3])};    \
      _Pragma("unroll") for (int dd = 0; dd < 4; ++dd) O[dd] *= alpha;                                     \
      _Pragma("unroll") for (int kh = 0; kh < 2; ++kh) {                                                   \
        /* selects, not pk[... + hl]: a lane-dependent index puts pk in scratch */                       \
        const uint2 mine = hl ? pk[2 * kh + 1] : pk[2 * kh], give = hl ? pk[2 * kh] : pk[2 * kh + 1];      \
        uint2 got;                                                                                         \
        got.x = __shfl_xor(give.x, 32, WAVE);                                                              \
        got.y = __shfl_xor(give.y, 32, WAVE);                                                              \
        const v4u pb = hl == 0 ? v4u{mine.x, mine.y, got.x, got.y} : v4u{got.x, got.y, mine.x, mine.y};    \
        _Pragma("unroll") for (int dd = 0; dd < 4; ++dd) {                                                 \
          const v4u vf = __builtin_bit_cast(v4u, S.v[(32 * dd + kk) * 4 + 2 * kh + hl]);                  \
          O[dd] = mfma32(vf, pb, O[dd]);                                                                   \
        }                                                                                                  \
      }                                                                                                    \
    }                                                                                                      \
  }
  PF_ISSUE(st0, 0);
  PF_ISSUE(st1, 1);
  int t = 0;
#define PF_STEP(SC, SI, t_)                                                                                \
  {                                                                                                        \
    PF_SYNC();                                                                                             \
    PF_TILE(SC, t_);                                                                                       \
    PF_ISSUE(SI, (t_) + 2);                                                                                \
  }
  for (; t + 2 < ntiles; t += 3) {
    PF_STEP(st0, st2, t);
    PF_STEP(st1, st0, t + 1);
    PF_STEP(st2, st1, t + 2);
  }
  if (t < ntiles) PF_STEP(st0, st2, t);
  if (t + 1 < ntiles) PF_STEP(st1, st0, t + 1);
#undef PF_STEP
#undef PF_TILE
#undef PF_SYNC
#undef PF_ISSUE
  __builtin_amdgcn_s_waitcnt(0);  // no direct load outlives the workgroup's LDS
  if (!cvalid) return;
  const float l_tot = l_run + __shfl_xor(l_run, 32, WAVE);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  // lane: column l % 32; register 4 i4 + x of O[dd] is dim 32 dd + 8 i4 + 4 hl + x
#pragma unroll
  for (int dd = 0; dd < 4; ++dd)
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      uint2 pk;
      pk.x = pack2bf(O[dd][4 * i4] * inv, O[dd][4 * i4 + 1] * inv);
      pk.y = pack2bf(O[dd][4 * i4 + 2] * inv, O[dd][4 * i4 + 3] * inv);
      *(uint2*)(y + frag_idx(base + j, head * HD + 32 * dd + 8 * i4 + 4 * hl, H * HD)) = pk;
    }
}

// One workgroup per (row, KV group, query block): merge the key splits of
// its 16 columns and normalise; thread t owns column t / 16 and 8
// consecutive dimensions.
template <typename T>
__global__ __launch_bounds__(256) void k_attn_combine(const float* __restrict__ part_o,
                                                      const float* __restrict__ part_ml, T* __restrict__ y, int H,
                                                      int G, int nqblk, int nsplit, const int* __restrict__ row_off,
                                                      int max_per_row, int Mcap) {
  constexpr int HD = 128;
  const int bg = blockIdx.x, qb = blockIdx.y;
  const int b = bg / G, g = bg - b * G, rep = H / G;
  const RowSpan sp = row_span(row_off, b, max_per_row, Mcap);
  const int base = sp.base, ncol = sp.n * rep;
  const int c = threadIdx.x >> 4, d0 = (threadIdx.x & 15) * 8;
  const int col = qb * 16 + c;
  if (col >= ncol) return;
  const int j = col / rep, head = g * rep + (col - j * rep);
  const int64_t pb = ((int64_t)bg * nqblk + qb) * nsplit;
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, part_ml[((pb + s) * 16 + c) * 2]);
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float L = 0.f;
  if (M != -INFINITY) {
    for (int s = 0; s < nsplit; ++s) {
      const float ms = part_ml[((pb + s) * 16 + c) * 2];
      if (ms == -INFINITY) continue;
      const float a = exp2f(ms - M);
      L += a * part_ml[((pb + s) * 16 + c) * 2 + 1];
      const float4* po = (const float4*)(part_o + ((pb + s) * 16 + c) * HD + d0);
      const float4 u0 = po[0], u1 = po[1];
      o[0] += a * u0.x; o[1] += a * u0.y; o[2] += a * u0.z; o[3] += a * u0.w;
      o[4] += a * u1.x; o[5] += a * u1.y; o[6] += a * u1.z; o[7] += a * u1.w;
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  // y is the c_proj GEMM's operand [token][H * 128]: 8 consecutive k are one
  // contiguous 16-byte group in both layouts
  T* yo = y + act_idx<T>(base + j, head * HD + d0, H * HD);
  if constexpr (sizeof(T) == 2) {
    uint4 pk;
    pk.x = (uint32_t)f2bf(o[0] * inv) | ((uint32_t)f2bf(o[1] * inv) << 16);
    pk.y = (uint32_t)f2bf(o[2] * inv) | ((uint32_t)f2bf(o[3] * inv) << 16);
    pk.z = (uint32_t)f2bf(o[4] * inv) | ((uint32_t)f2bf(o[5] * inv) << 16);
    pk.w = (uint32_t)f2bf(o[6] * inv) | ((uint32_t)f2bf(o[7] * inv) << 16);
    *(uint4*)yo = pk;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) st<T>(yo, i, o[i] * inv);
  }
}

// ---------------------------------------------------------------------------
// VALU attention, reference operation order (fp32 parity path, any hd <= 128)
// ---------------------------------------------------------------------------
#define VALU_MAXK 8192
template <typename T>
__global__ __launch_bounds__(256) void k_attn_valu(const T* __restrict__ q, const T* __restrict__ kc,
                                                   const T* __restrict__ vc, T* __restrict__ y, int H, int G, int hd,
                                                   int cap, const int* __restrict__ row_off,
                                                   const int* __restrict__ start, int max_per_row, int Mcap,
                                                   int window, float scale) {
  __shared__ float qs[128];
  __shared__ float sc[VALU_MAXK];
  __shared__ float red[16];
  const int j = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const RowSpan sp = row_span(row_off, b, max_per_row, Mcap);
  const int base = sp.base;
  if (j >= sp.n) return;
  const int m = base + j;
  const int rep = H / G, g = h / rep;
  const int pos = min(start[b] + j, cap - 1);
  const int lo = window > 0 ? max(0, pos - window) : 0;
  const int nk = min(pos - lo + 1, VALU_MAXK);
  const int64_t bg = (int64_t)b * G + g;
  for (int d = threadIdx.x; d < hd; d += blockDim.x) qs[d] = ld<T>(q, ((int64_t)m * H + h) * hd + d);
  __syncthreads();
  for (int i = threadIdx.x; i < nk; i += blockDim.x) {
    const T* kr = kc + (bg * cap + lo + i) * hd;
    float s = 0.f;
    for (int d = 0; d < hd; ++d) s += qs[d] * ld<T>(kr, d);
    sc[i] = s * scale;
  }
  __syncthreads();
  float mx = -INFINITY;
  for (int i = threadIdx.x; i < nk; i += blockDim.x) mx = fmaxf(mx, sc[i]);
  mx = block_max(mx, red);
  float sum = 0.f;
  for (int i = threadIdx.x; i < nk; i += blockDim.x) {
    const float e = expf(sc[i] - mx);
    sc[i] = e;
    sum += e;
  }
  sum = block_sum(sum, red);
  for (int i = threadIdx.x; i < nk; i += blockDim.x) sc[i] = sc[i] / sum;
  __syncthreads();
  const T* vb = vc + bg * (cap / 32) * hd * 32;
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float acc = 0.f;
    for (int i = 0; i < nk; ++i) {
      const int key = lo + i;
      acc += sc[i] * ld<T>(vb, ((int64_t)(key >> 5) * hd + d) * 32 + (key & 31));
    }
    st<T>(y, act_idx<T>(m, h * hd + d, H * hd), acc);
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
// Workgroups a typical attention launch is split into (key splits x rows x
// KV groups x query blocks).
#ifndef FC_ATTN_TARGET_WG
#define FC_ATTN_TARGET_WG 256
#endif
// query columns per row from which a chunk takes the prefill kernel
#ifndef FC_ATTN_CHUNK_COLS
#define FC_ATTN_CHUNK_COLS 128
#endif
// waves per attention workgroup (they take the block's 32-key tiles round robin)
#ifndef FC_ATTN_WAVES
#define FC_ATTN_WAVES 4
#endif

AttnGrid fc_attn_grid(int batch, int max_per_row, int typ_per_row, int n_head, int n_kv_head, int max_keys) {
  AttnGrid a;
  const int rep = n_head / n_kv_head;
  a.nqblk = (max_per_row * rep + 15) / 16;
  // split the key range so that the blocks a typical chunk fills reach ~4
  // workgroups per CU
  const int typ_blk = std::min(a.nqblk, std::max(1, (typ_per_row * rep + 15) / 16));
  // two query blocks per workgroup when a typical row x group fills more than one
  a.qb = typ_blk >= 2 ? 2 : 1;
  const int64_t units = (int64_t)batch * n_kv_head * ((typ_blk + a.qb - 1) / a.qb);
  const int range = max(max_keys, 1);
  int want = (int)((FC_ATTN_TARGET_WG + units - 1) / units);
  want = max(1, min(want, (range + 127) / 128));
  int sk = (range + want - 1) / want;
  sk = max(128, (sk + 127) / 128 * 128);
  a.split_keys = sk;
  a.nsplit = (range + sk - 1) / sk;
  return a;
}

int64_t fc_attn_part_bytes(int batch, int max_per_row, int n_head, int n_kv_head, int head_dim, int max_keys) {
  if (head_dim != 128) return 0;
  // fc_attn_grid never makes more splits than ceil(FC_ATTN_TARGET_WG /
  // units), and one token per row gives the fewest units
  AttnGrid a = fc_attn_grid(batch, max_per_row, 1, n_head, n_kv_head, max_keys);
  const int64_t units1 = (int64_t)batch * n_kv_head;
  const int64_t nsplit = std::max<int64_t>(a.nsplit, (FC_ATTN_TARGET_WG + units1 - 1) / units1);
  const int64_t units = (int64_t)batch * n_kv_head * a.nqblk * nsplit * 16;
  return fc_align(units * 128 * 4) + fc_align(units * 2 * 4);
}

// Prefill-width chunks (bf16, head_dim 128, >= FC_ATTN_CHUNK_COLS query
// columns per row and KV group) take k_attn_pf, which writes no partials.
static bool attn_uses_pf(int dtype, int hd, int typ_per_row, int H, int G) {
  return dtype == FC_BF16 && hd == 128 && G > 0 && typ_per_row * (H / G) >= FC_ATTN_CHUNK_COLS;
}

int fc_launch_attention(const void* q, const void* kc, const void* vc, void* y, int B, int max_tokens,
                        int max_per_row, int typ_per_row, int H, int G, int hd, int cap, const int* row_off,
                        const int* start, int window, int max_keys, int dtype, void* part, int64_t part_bytes,
                        hipStream_t s) {
  FC_CHECK_ARG(H % G == 0, "n_head must be a multiple of n_kv_head");
  FC_CHECK_ARG(cap % 32 == 0, "cache capacity must be a multiple of 32");
  FC_CHECK_ARG(max_per_row > 0, "max_per_row");
  const float scale = 1.f / sqrtf((float)hd);
  if (attn_uses_pf(dtype, hd, typ_per_row, H, G)) {
    FC_CHECK_ARG(B * G <= 65535, "batch * n_kv_head must be <= 65535");
    const int ncolmax = max_per_row * (H / G);
    // prefill-width chunks: 128 query columns per workgroup, 32x32x16 MFMA
    hipLaunchKernelGGL(k_attn_pf, dim3((ncolmax + 127) / 128, B * G), dim3(256), 0, s, (const bf16_t*)q,
                       (const bf16_t*)kc, (const bf16_t*)vc, (bf16_t*)y, H, G, cap, row_off, start, max_per_row,
                       max_tokens, window, scale * 1.4426950408889634f);
  } else if (dtype == FC_BF16 && hd == 128) {
    AttnGrid a = fc_attn_grid(B, max_per_row, typ_per_row, H, G, max_keys);
    const int64_t units = (int64_t)B * G * a.nqblk * a.nsplit * 16;
    FC_CHECK_ARG(part != nullptr && part_bytes >= fc_align(units * 128 * 4) + fc_align(units * 2 * 4),
                 "attention workspace too small");
    float* po = (float*)part;
    float* pml = (float*)((char*)part + fc_align(units * 128 * 4));
    FC_CHECK_ARG(B * G <= 65535, "batch * n_kv_head must be <= 65535");
    const float sl2 = scale * 1.4426950408889634f;
    if (a.qb == 2)
      hipLaunchKernelGGL((k_attn_mfma_qb<FC_ATTN_WAVES, 2>), dim3(a.nsplit, B * G, (a.nqblk + 1) / 2),
                         dim3(64 * FC_ATTN_WAVES), 0, s, (const bf16_t*)q, (const bf16_t*)kc, (const bf16_t*)vc, po,
                         pml, (bf16_t*)y, H, G, cap, row_off, start, max_per_row, max_tokens, window, a.split_keys,
                         a.nsplit, a.nqblk, sl2);
    else
      hipLaunchKernelGGL(k_attn_mfma<FC_ATTN_WAVES>, dim3(a.nsplit, B * G, a.nqblk), dim3(64 * FC_ATTN_WAVES),
                         0, s, (const bf16_t*)q, (const bf16_t*)kc, (const bf16_t*)vc, po, pml, (bf16_t*)y, H, G, cap,
                         row_off, start, max_per_row, max_tokens, window, a.split_keys, a.nsplit, a.nqblk, sl2);
    if (a.nsplit > 1) {
      FC_LAUNCH_CHECK();
      hipLaunchKernelGGL(k_attn_combine<bf16_t>, dim3(B * G, a.nqblk), dim3(256), 0, s, po, pml, (bf16_t*)y, H, G,
                         a.nqblk, a.nsplit, row_off, max_per_row, max_tokens);
    }
  } else {
    FC_CHECK_ARG(hd <= 128, "head_dim must be <= 128");
    FC_CHECK_ARG(max_keys <= VALU_MAXK, "VALU attention supports at most 8192 visible keys");
    const dim3 grid(max_per_row, H, B);
    if (dtype == FC_BF16)
      hipLaunchKernelGGL(k_attn_valu<bf16_t>, grid, dim3(256), 0, s, (const bf16_t*)q, (const bf16_t*)kc,
                         (const bf16_t*)vc, (bf16_t*)y, H, G, hd, cap, row_off, start, max_per_row, max_tokens,
                         window, scale);
    else
      hipLaunchKernelGGL(k_attn_valu<float>, grid, dim3(256), 0, s, (const float*)q, (const float*)kc,
                         (const float*)vc, (float*)y, H, G, hd, cap, row_off, start, max_per_row, max_tokens, window,
                         scale);
  }
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int64_t fc_attention_workspace_bytes(int32_t batch, int32_t max_per_row, int32_t n_head,
                                                int32_t n_kv_head, int32_t head_dim, int32_t max_keys) {
  return fc_attn_part_bytes(batch, max_per_row, n_head, n_kv_head, head_dim, max_keys);
}

extern "C" int32_t fc_attention(const void* q, const void* kc, const void* vc, void* y, int32_t batch,
                                int32_t max_tokens, int32_t max_per_row, int32_t n_head, int32_t n_kv_head,
                                int32_t head_dim, int32_t cap, const int32_t* row_off, const int32_t* start,
                                int32_t window, int32_t max_keys, int32_t dtype, void* work, int64_t work_bytes,
                                void* stream) {
  FC_CHECK_ARG(q && kc && vc && y && row_off && start, "null pointer");
  FC_CHECK_ARG(batch > 0 && max_tokens > 0 && max_per_row > 0 && n_head > 0 && n_kv_head > 0, "sizes");
  FC_CHECK_ARG(max_keys > 0 && max_keys <= cap, "max_keys must be in [1, cap]");
  return fc_launch_attention(q, kc, vc, y, batch, max_tokens, max_per_row, max_per_row, n_head, n_kv_head, head_dim,
                             cap, row_off, start, window, max_keys, dtype, work, work_bytes, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// fc_attention_noalloc: fc_attention for callers that cannot allocate (code
// under stream capture, serving loops that forbid allocation). The split-KV
// partials (unnormalised O and (max, sum) per query column and key split)
// live in `scratch`, a file-scope device array each GPU holds until the
// process ends. Nothing in it has to start at zero: a launch writes every
// partial its combine step reads (empty key splits write (-inf, 0)). All
// calls on one GPU share that GPU's array, so calls that overlap in time on
// one GPU (different streams, or host threads) race; calls ordered on one
// stream do not.
// ---------------------------------------------------------------------------
#ifndef FC_NOALLOC_SCRATCH_BYTES
#define FC_NOALLOC_SCRATCH_BYTES (32ll << 20)
#endif
static __device__ __align__(256) char scratch[FC_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchMaxDevices];  // device address of `scratch`, per device
}  // namespace

// The device address of `scratch` on the GPU `stream` runs on (the current
// device for the null stream), looked up once per device with that device
// current. Host code must use this address, never the array's name.
static int fc_scratch_ptr(hipStream_t stream, void** out) {
  int cur = 0;
  FC_HIP(hipGetDevice(&cur));
  int dev = cur;
  if (stream != nullptr) {
    hipDevice_t sd = 0;
    FC_HIP(hipStreamGetDevice(stream, &sd));
    dev = (int)sd;
  }
  FC_CHECK_ARG(dev >= 0 && dev < kScratchMaxDevices, "device ordinal beyond the scratch table");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur) FC_HIP(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) FC_HIP(hipSetDevice(cur));
    if (e != hipSuccess || p == nullptr) {
      fc_set_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
      return FC_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FC_OK;
}

// Resolves the scratch address of the stream's GPU ahead of time: fc_graph_begin
// calls it before capture starts, so a captured fc_attention_noalloc makes no
// runtime lookup inside the capture.
int fc_noalloc_prepare(hipStream_t stream) {
  void* p = nullptr;
  return fc_scratch_ptr(stream, &p);
}

extern "C" int64_t fc_attention_noalloc_max_bytes(void) { return FC_NOALLOC_SCRATCH_BYTES; }

extern "C" int32_t fc_attention_noalloc(const void* q, const void* kc, const void* vc, void* y, int32_t batch,
                                        int32_t max_tokens, int32_t max_per_row, int32_t n_head, int32_t n_kv_head,
                                        int32_t head_dim, int32_t cap, const int32_t* row_off, const int32_t* start,
                                        int32_t window, int32_t max_keys, int32_t dtype, void* stream) {
  FC_CHECK_ARG(q && kc && vc && y && row_off && start, "null pointer");
  FC_CHECK_ARG(batch > 0 && max_tokens > 0 && max_per_row > 0 && n_head > 0 && n_kv_head > 0, "sizes");
  FC_CHECK_ARG(max_keys > 0 && max_keys <= cap, "max_keys must be in [1, cap]");
  FC_CHECK_ARG(n_head % n_kv_head == 0, "n_head must be a multiple of n_kv_head");
  // the same kernel choice as fc_launch_attention (typical = max_per_row
  // here): only the split decode kernel (bf16, head_dim 128, below prefill
  // width) writes partials; the prefill and VALU kernels need none
  const bool split = dtype == FC_BF16 && head_dim == 128 &&
                     !attn_uses_pf(dtype, head_dim, max_per_row, n_head, n_kv_head);
  const int64_t need = split ? fc_attn_part_bytes(batch, max_per_row, n_head, n_kv_head, head_dim, max_keys) : 0;
  if (need > FC_NOALLOC_SCRATCH_BYTES) {
    fc_set_error("fc_attention_noalloc: these sizes need " + std::to_string(need) +
                 " bytes of split-KV partials; the static scratch holds " +
                 std::to_string((long long)FC_NOALLOC_SCRATCH_BYTES) + " (use fc_attention with a workspace)");
    return FC_ERR_CAPACITY;
  }
  void* part = nullptr;
  const int rc = fc_scratch_ptr((hipStream_t)stream, &part);
  if (rc != FC_OK) return rc;
  return fc_launch_attention(q, kc, vc, y, batch, max_tokens, max_per_row, max_per_row, n_head, n_kv_head, head_dim,
                             cap, row_off, start, window, max_keys, dtype, part, FC_NOALLOC_SCRATCH_BYTES,
                             (hipStream_t)stream);
}
