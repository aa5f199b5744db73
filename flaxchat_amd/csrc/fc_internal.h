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
