/*
 * flaxchat_amd: C-ABI of the MI355X (gfx950) speculative-decoding engine.
 *
 * Every entry point takes plain device pointers and sizes, enqueues work on
 * the HIP stream it is given (`stream` is a hipStream_t; NULL = the null
 * stream), allocates nothing, and returns FC_OK (0) or a negative status;
 * fc_last_error() then describes the failure. No C++ exception crosses the
 * boundary. The caller owns every buffer.
 *
 * The reference (mlnomadpy/flaxchat) has no native code: each entry point
 * below replaces a piece of eager JAX in flaxchat/engine.py or
 * flaxchat/gpt.py, cited on its declaration. The Python host
 * (flaxchat_amd/engine.py) keeps the reference's call surface,
 * generate_speculative() and generate_fast(), on top of this ABI.
 *
 * Layouts (row-major, C order, unless noted):
 *   Linear weights   [out][in]   (the transpose of Flax's (in, out) kernel); in
 *                    bf16 stored in fragment order (below), in fp32 row-major
 *   fragment order   of a bf16 matrix-core operand [R][K] (R padded to a
 *                    multiple of 16, K % 32 == 0): 16-row x 32-k blocks of
 *                    1 KB in [row block][k step] order; byte 16*l of a block
 *                    holds row l % 16, k = 8*(l/16) .. +7 of the step.
 *                    fc_pack_operand converts a row-major matrix.
 *   K cache          [layer][batch][kv_head][cap][head_dim]; with bf16 and
 *                    head_dim 128 (the matrix-core attention) each 32-position
 *                    block of 8 KB is in the fragment order of the K.Q^T
 *                    product: position 32 B + kk, dim d at element
 *                    B*4096 + ((2*(d/32) + (kk/4)%2)*64 + 4*(kk/8) + kk%4
 *                    + 16*((d/8)%4))*8 + d%8
 *   V cache          [layer][batch][kv_head][cap/32][head_dim][32]
 *                    (32-position blocks stored transposed so that the
 *                    P·V matrix-core operand is one 16-byte load per lane)
 *   smear history    [batch][cap][n_embd] fp32 (smeared embedding per position)
 *   chunk tokens     packed: row b feeds tokens[row_off[b]] .. tokens[row_off[b+1]-1]
 *                    at positions start[b], start[b]+1, ...; row_off[batch] is the
 *                    chunk's total, a device value (rows may feed nothing).
 *                    Per-token activations (q, y) are packed the same way.
 */
#ifndef FLAXCHAT_AMD_H
#define FLAXCHAT_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FC_OK 0
#define FC_ERR_ARG (-1)
#define FC_ERR_HIP (-2)
#define FC_ERR_UNSUPPORTED (-3)
#define FC_ERR_CAPACITY (-4)

#define FC_F32 0
#define FC_BF16 1

/* One transformer block's parameters (flaxchat/gpt.py:85-99, 154-163). */
typedef struct fc_layer {
  const void* wqkv;      /* [(H+2G)*hd][D]  c_q | c_k | c_v stacked on out   */
  const void* wo;        /* [D][H*hd]       attn.c_proj                       */
  const void* wfc;       /* [4D][D]         mlp.c_fc                          */
  const void* wproj;     /* [D][4D]         mlp.c_proj                        */
  const void* ve;        /* [Vp][G*hd] value embedding, NULL if none          */
  const float* ve_gate;  /* [G][12] fp32, NULL if none                        */
  int32_t window;        /* left window (> 0) or 0 for none                   */
  float resid_lambda;    /* resid_lambdas[i]                                  */
  float x0_lambda;       /* x0_lambdas[i]                                     */
} fc_layer;

/* A model (flaxchat/gpt.py:202-261). `layers` is a HOST array. */
typedef struct fc_model {
  int32_t n_layer, n_embd, n_head, n_kv_head, head_dim, vocab, vocab_pad, dtype;
  const void* wte;        /* [Vp][D]                                          */
  const void* lm_head;    /* [Vp][D] (== wte when tied)                       */
  const float* smear_gate;/* [24]                                             */
  float smear_lambda, backout_lambda;
  const float* rope_cos;  /* [rope_len][hd/2] fp32                            */
  const float* rope_sin;
  int32_t rope_len;
  const fc_layer* layers;
} fc_model;

/* Preallocated KV cache + smear history of one model. */
typedef struct fc_cache {
  void* k;
  void* v;
  float* hist;
  int32_t batch, cap;     /* cap is a multiple of 32                          */
} fc_cache;

/* One chunk of tokens per row, fed at per-row positions (packed layout
 * above). The capacities size the grids and the workspace; kernel shapes
 * are tuned for typ_tokens. */
typedef struct fc_chunk {
  int32_t max_tokens;     /* capacity: row_off[batch] <= max_tokens           */
  int32_t max_per_row;    /* no row feeds more tokens (<= 1024)               */
  int32_t typ_tokens;     /* typical total (0: max_tokens)                    */
  const int32_t* tokens;  /* [max_tokens]  device, packed                     */
  const int32_t* row_off; /* [batch+1]     device, row_off[0] == 0            */
  const int32_t* start;   /* [batch]       device, position of the first token */
  int32_t n_out;          /* logits for the last n_out tokens of each row     */
  float* logits;          /* row (b, r) at logits + b*logits_stride + r*V;    */
                          /* unspecified for a row with fewer than n_out tokens */
  int64_t logits_stride;  /* floats between rows b and b+1                    */
  int32_t flags;          /* FC_CHUNK_* bits; 0 = the per-token decode forward  */
} fc_chunk;

/* fc_chunk.flags: smear as the full-sequence forward GPT.__call__ does
 * (flaxchat/gpt.py:418-421): x_t = n_t + gate_t * n_{t-1} with n the
 * normalised embeddings, where the per-token decode forward
 * (flaxchat/engine.py:84-87) adds gate_t * x_{t-1}, the previous smeared
 * value. The cache's smear history then holds n for the next chunk. */
#define FC_CHUNK_FULL_SMEAR 1

/* Per-row sampling statistics of a logits row (see fc_row_stats). */
typedef struct fc_rowstat {
  float mx;        /* max over kept entries of z/T                           */
  float sum;       /* sum over kept entries of exp(z/T - mx)                 */
  float tau;       /* top-k threshold value (-inf when top-k is off)         */
  int32_t tie_idx; /* entries equal to tau are kept iff index <= tie_idx     */
  int32_t argmax;  /* first index of the maximum                             */
  int32_t pad[3];
} fc_rowstat;

/* Device state of a speculative-decoding batch (one row per sequence).
 * All pointers are device int32 arrays sized as noted; the host fills
 * them once after prefill and then only reads `result` and `gen`. */
typedef struct fc_spec_state {
  int32_t batch, k, max_tokens, gen_cap, vocab;
  float temperature;      /* <= 0: greedy                                      */
  int32_t top_k;          /* <= 0: off                                         */
  uint64_t seed;
  int32_t* t_len;  int32_t* d_len;       /* [B] cache lengths                  */
  int32_t* t_pend; int32_t* d_pend;      /* [B][FC_PMAX] pending tokens        */
  int32_t* t_pend_n; int32_t* d_pend_n;  /* [B]                                */
  int32_t* t_dirty; int32_t* d_dirty;    /* [B] earliest fed != emitted pos    */
  int32_t* gen;    int32_t* gen_n;       /* [B][gen_cap] tokens incl. prompt   */
  int32_t* prompt_len;                   /* [B]                                */
  int32_t* round;                        /* [B] round counter (Philox)         */
  int32_t* stall;                        /* [B] nonzero: row re-feeds a rollback */
                                         /* backlog longer than FC_PMAX           */
  int32_t* result;                       /* [B][FC_RES_STRIDE]                 */
  /* per-round scratch (chunks in the packed layout) */
  int32_t* tok_d0;   /* [B*FC_PMAX]     draft step 0 tokens                    */
  int32_t* off_d0;   /* [B+1]                                                  */
  int32_t* start_d;  /* [k][B]          draft step start positions             */
  int32_t* tok_ds;   /* [k][B]          draft step tokens (steps 1..k-1)       */
  int32_t* off_ds;   /* [B+1]           rows fed at steps 1..k-1               */
  int32_t* tok_v;    /* [B*(FC_PMAX+k)] verify chunk tokens                    */
  int32_t* off_v;    /* [B+1]                                                  */
  int32_t* start_v;  /* [B]                                                    */
  int32_t* drafts;   /* [B][k]                                                 */
  float* q_logits;   /* [B][k][V]                                              */
  float* p_logits;   /* [B][k+1][V]                                            */
  fc_rowstat* q_stats; /* [B][k]                                               */
  fc_rowstat* p_stats; /* [B][k+1]                                             */
  void* part;          /* vocab-pass partials, fc_spec_part_bytes(batch, k, vocab) */
  int64_t part_bytes;
} fc_spec_state;

#define FC_RES_STRIDE 40
#define FC_PMAX 16
/* Tokens a model still has to be fed (fed next round ahead of the drafts):
 * normally 1 (target) or 1-2 (draft); after a rejection that rolls back past
 * a stale cache entry, up to FC_PMAX. A longer rollback stalls the row: the
 * following rounds re-feed FC_PMAX tokens of each model's backlog
 * gen[len, gen_n - 1) per round, without drafting, until both caches hold
 * everything before gen_n - 1 (stall[b] then returns to 0). Result row
 * layout: [0] n_emitted this round, [1] accepted, [2] rejected index or -1,
 * [3] flags (bit0 the rollback stalled the row; bit2 row finished; bit3 the
 * row was stalled this round: backlog re-fed, nothing emitted), [4] k',
 * [5] target pending count, [6] draft pending count, [8..8+k+1] emitted
 * tokens. */

const char* fc_last_error(void);
int32_t fc_version(void);

/* Bytes of workspace fc_forward needs for chunks with these capacities. */
int64_t fc_forward_workspace_bytes(const fc_model* m, int32_t batch, int32_t max_tokens,
                                   int32_t max_per_row, int32_t typ_tokens);

/* Feed one chunk through the model: embedding + smear, every block, head.
 * Replaces the per-token `_single_step_forward` (flaxchat/engine.py:51-177)
 * and the token-by-token `_prefill` (flaxchat/engine.py:396-407) with one
 * batched multi-token pass; appends K/V at each valid slot's position. */
int32_t fc_forward(const fc_model* m, const fc_cache* c, const fc_chunk* ch,
                   void* work, int64_t work_bytes, void* stream);

/* GEMM with fused epilogue: out[M][N] = epi(A[M][K] . W[N][K]^T), A and W in
 * `dtype`. Replaces the nnx.Linear matmuls of flaxchat/engine.py:106-108,
 * 158, 161, 172 (flaxchat/gpt.py:93-99, 154-163). epi: 0 store fp32,
 * 1 add into fp32 out, 2 relu^2 (flaxchat/gpt.py:161) stored in `dtype`,
 * 4 15*tanh(z/15) softcap (flaxchat/engine.py:173-174) stored fp32.
 * bf16: A, W and a bf16 relu^2 output are in fragment order (A padded to
 * round16(M) rows), K % 64 == 0, N % 32 == 0; fp32: all row-major. */
int32_t fc_gemm(const void* A, const void* W, void* out, int32_t M, int32_t N, int32_t K,
                int32_t dtype, int32_t epi, void* stream);

/* Fragment-order copy of a row-major bf16 matrix src[rows][K] into
 * dst[round16(rows)][K] (padding rows zero). No reference counterpart: the
 * layout change of the bf16 weights and GEMM operands. */
int32_t fc_pack_operand(const void* src, void* dst, int32_t rows, int32_t K, void* stream);

/* Split-KV flash-decode attention over a cache layer (flaxchat/engine.py:128-156):
 * GQA head grouping, causal + inclusive sliding window `pos - j <= window`.
 * q: [max_tokens][H][hd] dtype, packed (row_off, start as in fc_chunk);
 * y: [max_tokens][H*hd] dtype (bf16: fragment order over round16(max_tokens)
 * rows); rows past row_off[batch] untouched. A row whose tokens run past
 * max_tokens or number more than max_per_row is treated as empty. */
int64_t fc_attention_workspace_bytes(int32_t batch, int32_t max_per_row, int32_t n_head, int32_t n_kv_head,
                                     int32_t head_dim, int32_t max_keys);
int32_t fc_attention(const void* q, const void* kc, const void* vc, void* y,
                     int32_t batch, int32_t max_tokens, int32_t max_per_row, int32_t n_head,
                     int32_t n_kv_head, int32_t head_dim, int32_t cap, const int32_t* row_off,
                     const int32_t* start, int32_t window, int32_t max_keys, int32_t dtype, void* work,
                     int64_t work_bytes, void* stream);

/* fc_attention without the workspace argument: the split-KV partials live in
 * a static device array of the library, fc_attention_noalloc_max_bytes()
 * bytes (32 MiB), which each GPU the library runs on holds until the process
 * ends. No counterpart in the reference: for callers that cannot allocate
 * (code under stream capture, serving loops, harnesses that forbid
 * hipMalloc). Same arguments and result as fc_attention; sizes whose
 * partials (fc_attention_workspace_bytes; none for fp32, nor at prefill
 * width: bf16 head_dim 128 with >= 128 query columns per row and KV group) exceed the
 * array return FC_ERR_CAPACITY before anything is launched. Every call on one
 * GPU shares that GPU's array: calls that overlap in time on one GPU race.
 * The array's device address is looked up once per GPU, at the first call
 * or at fc_graph_begin on a stream of that GPU: a caller that captures with
 * its own hipStreamBeginCapture makes one uncaptured call first. */
int64_t fc_attention_noalloc_max_bytes(void);
int32_t fc_attention_noalloc(const void* q, const void* kc, const void* vc, void* y,
                             int32_t batch, int32_t max_tokens, int32_t max_per_row, int32_t n_head,
                             int32_t n_kv_head, int32_t head_dim, int32_t cap, const int32_t* row_off,
                             const int32_t* start, int32_t window, int32_t max_keys, int32_t dtype,
                             void* stream);

/* Attention prologue of one layer for M packed tokens (flaxchat/engine.py:96-126,
 * flaxchat/gpt.py:52-71; the piece fc_forward runs between the QKV GEMM and the
 * attention). qkv: the QKV GEMM output, fp32 [M][(H + 2G) * head_dim] (q heads,
 * then k, then v). q and k heads: RoPE at position tok_pos[m] (the model's
 * tables), then 1.2 * RMSNorm (eps 1e-6). v heads of a layer with a value
 * embedding: v + 3 sigmoid(h[m][0:12] . ve_gate[g]) * ve[tokens[m]][g]. h is the
 * QKV GEMM's input (bf16: fragment order over round16(M) rows; fp32: row-major
 * [M][n_embd]). q -> q[m][H][head_dim] in the model dtype; k and v are written
 * into row tok_row[m] (< batch) of the layer's cache at tok_pos[m] when it lies
 * in [0, cap); tokens with tok_row[m] outside [0, batch) are skipped. */
int32_t fc_attn_prologue(const fc_model* m, int32_t layer, const fc_cache* c, const float* qkv,
                         const void* h, const int32_t* tokens, const int32_t* tok_row,
                         const int32_t* tok_pos, int32_t M, void* q, void* stream);

/* QKV projection of one layer followed by its attention prologue
 * (flaxchat/engine.py:96-126: the c_q / c_k / c_v matmuls of :106-108, then
 * what fc_attn_prologue does) for M tokens: h is the normalised input (bf16:
 * fragment order over round16(M) rows; fp32: row-major [M][n_embd]); q, the
 * cache writes and the skipped tokens as in fc_attn_prologue. For bf16,
 * head_dim 128 and verify / prefill row counts (typ_tokens, 0 = M) the
 * prologue runs in the GEMM's epilogue and no workspace is used; otherwise
 * the fp32 projection goes to `work` (fc_attn_qkv_workspace_bytes). */
int64_t fc_attn_qkv_workspace_bytes(const fc_model* m, int32_t M, int32_t typ_tokens);
int32_t fc_attn_qkv(const fc_model* m, int32_t layer, const fc_cache* c, const void* h,
                    const int32_t* tokens, const int32_t* tok_row, const int32_t* tok_pos, int32_t M,
                    int32_t typ_tokens, void* q, void* work, int64_t work_bytes, void* stream);

/* Per-row statistics of fp32 logits rows (flaxchat/engine.py:461-476):
 * lax.top_k keep-set (exactly k, lower index first among ties), max and
 * softmax normaliser of z/T over it, and the first-index argmax. */
int32_t fc_row_stats(const float* logits, int32_t rows, int32_t V, float temperature,
                     int32_t top_k, fc_rowstat* stats, void* stream);

/* One speculative round on device (flaxchat/engine.py:484-606 with the
 * sequential verify replaced by one (pending + k)-token verify chunk and the
 * re-prefill replaced by length-pointer rollback): draft k steps, verify,
 * accept/reject with residual resampling, bonus, bookkeeping. Every launch
 * shape is fixed by (batch, k), so one captured graph replays every round. */
int64_t fc_spec_workspace_bytes(const fc_model* target, const fc_model* draft, int32_t batch, int32_t k);
int32_t fc_spec_round(const fc_model* target, const fc_cache* tcache,
                      const fc_model* draft, const fc_cache* dcache,
                      const fc_spec_state* st, void* work, int64_t work_bytes, void* stream);

/* Bytes of fc_spec_state.part: per-chunk partials of the vocab-wide passes
 * (row statistics and Gumbel-max draws split over many workgroups). */
int64_t fc_spec_part_bytes(int32_t batch, int32_t k, int32_t vocab);

/* Accept/reject step alone on given logits (flaxchat/engine.py:525-592);
 * updates the state like fc_spec_round does. */
int32_t fc_spec_accept(const fc_spec_state* st, void* stream);

/* generate_fast sampling step (flaxchat/engine.py:308-324, 343-368): for
 * rows with !done[b] && pos[b] < max_pos[b], sample from logits row b,
 * write it at gen[b][pos[b]+1] and tok_cur[b], advance pos and step, set
 * done on eos. */
int32_t fc_fast_sample(const float* logits, int32_t batch, int32_t V, float temperature,
                       int32_t top_k, uint64_t seed, int32_t eos, int32_t* gen, int32_t gen_cap,
                       int32_t* pos, int32_t* done, int32_t* step, const int32_t* max_pos,
                       int32_t* tok_cur, fc_rowstat* stats, void* stream);

/* Engine.generate's token choice for one step (flaxchat/engine.py:666-683
 * sampling, :773-790 forced-or-sampled selection). For every row b:
 * forced[b] >= 0 takes that token (a tool-output token the caller queued;
 * the caller guarantees forced[b] < V); otherwise sample from logits row b
 * exactly as fc_fast_sample (argmax when temperature <= 0; top_k <= 0 keeps
 * the whole vocabulary; Philox counter (group, b, step[b])). The token is
 * written at gen[b][pos[b]+1] and tok_cur[b]; pos and step advance. Rows
 * never stop here: the reference's completion (assistant_end / bos) is the
 * caller's bookkeeping. */
int32_t fc_engine_sample(const float* logits, int32_t batch, int32_t V, float temperature,
                         int32_t top_k, uint64_t seed, const int32_t* forced, int32_t* gen,
                         int32_t gen_cap, int32_t* pos, int32_t* step, int32_t* tok_cur,
                         fc_rowstat* stats, void* stream);

/* Cross-entropy of GPT.__call__(idx, targets) (flaxchat/gpt.py:446-452):
 * for each of `rows` logits rows (row r at logits + r * row_stride, V
 * entries), loss[r] = logsumexp(z) - z[target[r]] in fp32, or 0 when
 * target[r] < 0 (masked); target[r] >= V is an error the caller excludes. */
int32_t fc_cross_entropy(const float* logits, int64_t row_stride, const int32_t* targets, int32_t rows,
                         int32_t V, float* loss, void* stream);

/* Streaming read of `bytes` (a multiple of 16) from device memory by
 * `workgroups` workgroups of 256 threads, each streaming one contiguous
 * share with 16-byte non-temporal loads; out receives 4 * workgroups
 * xor-folded words. No counterpart in the reference:
 * the benchmark's measured read ceiling, against which the HBM-bound kernels
 * are rated next to the 8 TB/s peak. */
int32_t fc_read_probe(const void* src, int64_t bytes, uint32_t* out, int32_t workgroups, void* stream);

/* Read of L2-resident data: workgroup w (256 threads) reads
 * bytes / workgroups bytes (rounded down to 64 KB) from the region of
 * `region_bytes` at src + (w % 8) * region_bytes (workgroups go to the
 * eight XCDs round robin, so each XCD's L2 holds one region; src must hold
 * 8 * region_bytes), wrapping, with direct global-to-LDS loads, sixteen 1 KB
 * loads in flight per wave; out receives 4 * workgroups words. No
 * counterpart in the reference: the ceiling against which the GEMMs'
 * L2-to-CU traffic is rated (MI355X: 4 MB of L2 per XCD). */
int32_t fc_l2_read_probe(const void* src, int64_t region_bytes, int64_t bytes, uint32_t* out, int32_t workgroups,
                         void* stream);

/* The decode attention's load pattern without its compute: workgroup u of
 * `units` reads the `tiles` consecutive 16 KB tiles at src + u * tiles *
 * 16384 (src must hold units * tiles * 16384 bytes), each of its four waves
 * taking every fourth tile as sixteen 1 KB non-temporal loads, as
 * k_attn_mfma walks a (row, KV group)'s K and V blocks; out receives
 * 256 * units words. No counterpart in the reference: the rate the verify
 * attention can reach with its grid and tile walk. */
int32_t fc_walk_probe(const void* src, int32_t units, int32_t tiles, uint32_t* out, void* stream);

/* A GEMM's operand walk without its arithmetic: for output tiles of
 * tile_m x tile_n (multiples of 16; tile_n divides N), K a multiple of 64
 * and a K split of `splits` (at most K / 64), each workgroup loads its
 * tile's 1 KB fragment-order blocks of W (N x K) and A (round16(M) x K)
 * over its split's 64-deep k chunks, four waves taking every fourth chunk,
 * 16 loads of 1 KB in flight per wave and no barrier,
 * the M tiles that share a weight slab on one XCD, as the K-split,
 * LDS-shared and ring GEMM kernels read them: with direct global-to-LDS
 * loads (reg_loads = 0; each wave's word is the XOR of its last 16 landed
 * blocks) or loads into registers (reg_loads = 1; the XOR of every block it
 * loaded). `out` receives fc_gemm_walk_probe_words(M, N, tile_m, tile_n,
 * splits) words (untouched for workgroups past the tiles). No counterpart
 * in the reference: the rate a GEMM of that tiling can reach whatever its
 * MFMA work and epilogue. */
int32_t fc_gemm_walk_probe(const void* A, const void* W, int32_t M, int32_t N, int32_t K, int32_t tile_m,
                           int32_t tile_n, int32_t splits, int32_t reg_loads, uint32_t* out, void* stream);
int32_t fc_gemm_walk_probe_words(int32_t M, int32_t N, int32_t tile_m, int32_t tile_n, int32_t splits);

/* Stream capture into a replayable hipGraph (the captured draft loop). */
int32_t fc_graph_begin(void* stream);
int32_t fc_graph_end(void* stream, void** exec_out);
int32_t fc_graph_launch(void* exec, void* stream);
int32_t fc_graph_destroy(void* exec);

#ifdef __cplusplus
}
#endif
#endif
