// Internal (not exported) declarations shared by the .hip translation units.
#pragma once
#include "fc_common.h"
#include <algorithm>

enum { EPI_STORE = 0, EPI_ADD = 1, EPI_RELU2 = 2, EPI_MLPOUT = 3, EPI_SOFTCAP = 4, EPI_PARTIAL = 5, EPI_QKV = 6 };

// EPI_QKV: the c_q|c_k|c_v GEMM finishes each (token, head) itself: RoPE +
// 1.2 RMSNorm for q / k heads, value-embedding gate for v heads, q written
// [M][H][128] bf16, k / v appended to the layer's cache (what k_prologue
// does after a plain GEMM).
struct QkvEpi {
  const int *tokens, *tok_row, *tok_pos;
  const float *rcos, *rsin;
  int rope_len;
  const uint16_t* ve;     // [Vp][G*128] or NULL
  const float* ve_gate;   // [G][12]
  const uint16_t* h;      // the GEMM's A operand (fragment order), for the gate
  int D, H, G, B, cap;
  uint16_t *kc, *vc, *q;  // layer's K / V cache, q output
};

// Vocab-pass partials of one logits row over one range of its entries
// (a chunk of the separate pass, or a column tile of the lm_head GEMM)
struct VPart {
  float zmax; int zarg;  // argmax of z (first index among equals)
  float m, s;            // max of x = z / T and sum of exp(x - m)
  float a; int ai;       // max of x - m + G, and its index
  float g; int gi;       // max of G, and its index
};

struct Epi {
  int mode;
  int out_dtype;
  void* out;
  int64_t ldo;
  // EPI_MLPOUT: out is x (fp32, in place)
  const float* x0;
  float* xb;
  float r, a, lb;
  int capture, last;
  // EPI_SOFTCAP: output row m -> (m / n_out) * row_stride + (m % n_out) * V
  int n_out;
  int64_t row_stride;
  int V;
  // EPI_SOFTCAP given `vp` (the LDS-shared kernel only): also the vocab-pass
  // partials of output row m over the tile's columns, vp[m * vp_ld + column
  // tile], at temperature vp_T (> 0: max / exp-sum of z / T, and with
  // vp_draw the Gumbel-max terms of Philox counter (column / 4, m,
  // vp_round[m], vp_slot) under key vp_seed; else the argmax alone)
  VPart* vp;
  int vp_ld, vp_draw, vp_slot;
  float vp_T;
  uint64_t vp_seed;
  const int* vp_round;
  // EPI_PARTIAL: split `split` writes part[(split * part_rows + m) * ldo + n]
  float* part;
  int part_rows, split;
  QkvEpi qkv;
  // The attention-side RMSNorm folded into the GEMMs (bf16; flaxchat/gpt.py:44-46,
  // engine.py:160-161): EPI_ADD given `xa` (unsplit, K-split kernel) also
  // writes bf16(new x) in fragment order to xa, the c_fc operand, and for
  // row m and its column tile nt the sum of squares of the new x over the
  // tile to ssq[nt * ssq_ld + m]; a GEMM given `rms_in` multiplies output row
  // m by 1 / sqrt(sum_{t < rms_n} rms_in[t * ssq_ld + m] / K + 1e-6) (summed in
  // a fixed order).
  uint16_t* xa;
  float* ssq;
  const float* rms_in;
  int ssq_ld, rms_n;
};

#define FC_MAX_SPLIT 8
// split-K partials of GEMMs writing the residual stream (finished by RMSNorm)
struct GemmWork {
  float* part;
  int64_t part_bytes;
};
int64_t fc_gemm_part_bytes(int Mtyp, int Mcap, int N, int K, int dtype);
// column tiles of the EPI_ADD GEMM that writes `xa` (the rms_n of its consumer),
// and whether its consumers can take that many
int fc_gemm_fold_tiles(int Mtyp, int N);
bool fc_gemm_fold_ok(int Mtyp, int D);
// `splits` (may be NULL: no split) receives the split count; when > 1 the
// output was written as partials to gw.part and the caller must finish it.
// true when the GEMM of this shape runs the tile that can finish the
// attention prologue in its epilogue (EPI_QKV; 128-column tiles, bf16)
bool fc_gemm_fuses_qkv(int Mtyp, int N, int K, int dtype, int head_dim);
int fc_launch_gemm(const void* A, const void* W, int Mcap, const int* Mdev, int Mtyp, int N, int K, int dtype,
                   const Epi& e, const GemmWork& gw,
                   hipStream_t s, int* splits);
// column tiles per row of an unsplit EPI_SOFTCAP GEMM of this shape when its
// kernel can write the vocab-pass partials (Epi::vp), else 0
int fc_gemm_vocab_tiles(int M, int N, int K, int dtype);
// fc_forward whose logits GEMM also writes the vocab-pass partials where its
// kernel can (see Epi::vp; `vp` may be NULL): *nch = partials per logits row
// then, else 0 (the caller runs the separate pass). `vp_cap` = VParts at vp;
// a GEMM with more than `max_tiles` column tiles is left to the separate pass.
struct VocabFuse {
  VPart* vp;
  int64_t vp_cap;
  int max_tiles;
  float T;
  int draw, slot;
  uint64_t seed;
  const int* round;
};
// The previous draft step's finish (fc_vocab.h draft_merge_row), which the
// embedding kernel of a one-token-per-row bf16 draft chunk can run itself
// (fc_embed_merges): row b's token is the merged draft of step `step`.
struct DraftMerge {
  const VPart* part;
  int nch;
  fc_rowstat* q_stats;
  int *drafts, *tok_v, *tok_ds;
  const int *off_v, *off_ds;
  int B, k, V, step;
  float T;
};
bool fc_embed_merges(const fc_model* m, const fc_chunk* ch);
int fc_forward_vp(const fc_model* m, const fc_cache* c, const fc_chunk* ch, void* work, int64_t work_bytes,
                  void* stream, const VocabFuse* vp, int* nch, const DraftMerge* dm = nullptr);

struct AttnGrid {
  int nqblk, nsplit, split_keys;
  int qb;  // query blocks per workgroup (1 or 2)
};
AttnGrid fc_attn_grid(int batch, int max_per_row, int typ_per_row, int n_head, int n_kv_head, int max_keys);
int64_t fc_attn_part_bytes(int batch, int max_per_row, int n_head, int n_kv_head, int head_dim, int max_keys);
int fc_launch_attention(const void* q, const void* kc, const void* vc, void* y, int B, int max_tokens,
                        int max_per_row, int typ_per_row, int H, int G, int hd, int cap, const int* row_off,
                        const int* start, int window, int max_keys, int dtype, void* part, int64_t part_bytes,
                        hipStream_t s);
// fc_attention_noalloc's scratch address for the stream's GPU, looked up now
// (fc_graph_begin runs it before a capture starts)
int fc_noalloc_prepare(hipStream_t stream);
int fc_launch_prologue(const float* qkv, const void* h, const int* tokens, const fc_model* m, int layer,
                       const fc_cache* c, const int* tok_row, const int* tok_pos, int Mcap, const int* Mdev, void* q,
                       hipStream_t s);
int fc_launch_row_stats(const float* logits, int rows, int V, float T, int top_k, fc_rowstat* stats, hipStream_t s);
