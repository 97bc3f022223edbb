/* libaneforge_hip: the C ABI of the MI355X (gfx950) quantized-decode path.
 *
 * This library replaces the native layer the reference binds through ctypes
 * (aneforge/_runtime.py:60-92 over aneforge/_lib/ane_e5rt_dispatch.mm:528-713).  The
 * reference hands a whole compiled ANE program to Espresso; here the same work is exposed as
 * kernel-level entry points that the Python host (aneforge_amd) sequences and captures into
 * HIP graphs.
 *
 * Conventions (all entry points):
 *   - return 0 on success, a negative code on failure; afx_last_error() gives the calling
 *     thread's message (reference: int rc / NULL handle + stderr, ane_e5rt_dispatch.mm:528).
 *   - every buffer is caller-owned DEVICE memory; nothing here allocates in the hot path.
 *   - fp16 buffers are raw IEEE-754 half bits; int8/Q4 codes are raw bytes.
 *   - `stream` is a hipStream_t (NULL = default stream); calls enqueue and return at once.
 *     The Python Program.execute() synchronises, preserving the reference's synchronous
 *     execute (ane_e5rt_dispatch.mm:667-673).
 *   - weight formats: 0 = int8 codes [N][K] + fp16 row scale [N]
 *                     1 = Q4_0 superblock codes [N][K/2] + fp16 block scales [N][K/32]
 *                     2 = fp16 [N][K]
 */
#ifndef ANEFORGE_HIP_H
#define ANEFORGE_HIP_H

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime plumbing --------------------------------------------------------------- */

/* Error text of the last failing call on this thread (reference: stderr text after rc -1,
 * aneforge/_lib/ane_e5rt_dispatch.mm:528-608). */
const char* afx_last_error(void);
int afx_abi_version(void);
/* CU count, LDS and L2 bytes, gfx arch number (reference: per-family limits tables,
 * aneforge/_targets.py:106-116, consulted before compiling). */
int afx_device_info(int device, int* cu_count, int* lds_bytes, int* l2_bytes, int* gcn_arch);
/* Block until `stream` drains (reference: synchronous execute, ane_e5rt_dispatch.mm:667-673). */
int afx_stream_sync(void* stream);
/* Capture a kernel sequence on `stream` into a replayable graph (reference: a compiled program
 * executed repeatedly, ane_e5rt_program_compile :528 / _execute :667). */
int afx_graph_begin(void* stream);
int afx_graph_end(void* stream, void** exec_out);
int afx_graph_launch(void* exec, void* stream);
/* (reference: ane_e5rt_program_release, ane_e5rt_dispatch.mm:675-677) */
int afx_graph_destroy(void* exec);
/* Events on the caller's stream, for timing the stream the kernels run on. */
int afx_event_create(void** ev);
int afx_event_record(void* ev, void* stream);
int afx_event_elapsed_ms(void* start, void* stop, float* ms);
int afx_event_destroy(void* ev);

/* ---- weight-streaming linear layers --------------------------------------------------- */

/* y[M][N] = x[M][K] @ W^T (+bias) (+residual, may alias y); out_f32 selects fp32 y.  Any M:
 * 4+ rows without a norm prologue run on MFMA, otherwise the vector kernels take 8 rows a launch.
 * ws (optional, device, may be NULL): an fp32 workspace of ws_bytes; with up to 32 * M * N bytes,
 * int8 / blockwise / fp16 rows too long for one pass of the persistent MFMA kernel (K above 4096
 * int8, 2048 fp16, at 16 or fewer rows) are cut into up to 8 K slices (as many as the workspace
 * holds at 4 * M * N bytes each) whose partials meet there, then a second launch sums them.  Dense
 * Q4_0 is measured faster unsplit and ignores ws.  Results differ from the single-pass kernels only
 * in fp32 summation order.
 * fmt 0: the compress="int8" linear, constexpr_affine_dequantize(axis=0) + matmul
 * (aneforge/_compile.py:171-179, 375-385; aneforge/graph.py:187-195); 1: the GGUF Q4_0 weights
 * the reference dequantises on the host and casts to fp16 (aneforge/_gguf.py:34-39), weight
 * fp16((code - 8) * d); 2: fp16; 3: compress=
 * "blockwise" with 32-weight blocks, int8 codes + fp16 scale[N][K/32], weight fp16(q * s)
 * (aneforge/_blob.py:46-56, constexpr_blockwise_shift_scale in aneforge/_compile.py:112-188);
 * 4: compress="int4", palettize_lut4's packed indices [N][K/2] (column 2j in the low nibble of byte
 * j) + a 16-entry fp16 codebook per row scale[N][16], weight codebook[n][index] (aneforge/_blob.py:
 * 28-43, constexpr_lut_to_dense in aneforge/_compile.py:149; vector kernels at any M);
 * 5: GGUF Q4_K after afx_q4_k_repack, weight fp16(d*sc*q - dmin*m) as the reference's
 * GGUFView.get produces it (aneforge/_gguf.py:34-39; K % 256 == 0, vector kernels at any M);
 * 6: GGUF Q6_K after afx_q6_k_repack, weight fp16(d*sc * (q - 32)) (the same reference path). */
int afx_linear(int fmt, const void* w, const void* scale, const void* x, int ldx, void* y, int ldy,
               int M, int N, int K, const void* bias, const void* residual, int out_f32,
               int rows_hint, void* ws, long long ws_bytes, void* stream);
/* y = rms_norm(x, gamma, eps) @ W^T (+bias): RMSNorm (aneforge/graph.py:293-301,
 * aneforge/_compile.py:738-755) fused as the GEMV prologue. */
int afx_linear_rms(int fmt, const void* w, const void* scale, const void* x, int ldx, const void* gamma,
                   float eps, void* y, int ldy, int M, int N, int K, const void* bias, int out_f32,
                   int rows_hint, void* stream);
/* The lm_head for one hidden row (aneforge/llm.py:338-404, the fp16 head): logits[N] (fp32) =
 * rms_norm(x, gamma, eps) @ W^T (fmt 2, W fp16 [N][K]), plus slots (16-byte aligned float4
 * [ceil(N/8)]): for rows 8s..8s+7, {largest logit, its row as int bits (lowest on ties), second
 * largest, largest |logit|}, which afx_decode_advance merges for the greedy pick and its tie margin;
 * and, if hn_out is not NULL, the fp16 normalised row the products used [K]. */
int afx_lm_head(int fmt, const void* w, const void* scale, const void* x, const void* gamma, float eps,
                float* logits, int N, int K, float* slots, void* hn_out, void* stream);
/* act[M][N/2] = silu(g) * u, rows of W interleaved (gate_i, up_i), optional RMSNorm first:
 * the front half of _swiglu (aneforge/llm.py:171-175). */
int afx_linear_swiglu(int fmt, const void* w, const void* scale, const void* x, int ldx, const void* gamma,
                      float eps, int norm, void* act, int ld_act, int M, int N, int K, int rows_hint,
                      void* stream);
/* act[M][N/2] = gelu_tanh(g) * u, otherwise as afx_linear_swiglu: the front half of _geglu, Gemma's
 * MLP (aneforge/llm.py:185-196; gelu_tanh is the reference's _gelu_tanh, llm.py:185-189). */
int afx_linear_geglu(int fmt, const void* w, const void* scale, const void* x, int ldx, const void* gamma,
                     float eps, int norm, void* act, int ld_act, int M, int N, int K, int rows_hint,
                     void* stream);
/* [q|k|v] = rms_norm(h) @ Wqkv^T (+bias), RoPE on q and k, k/v written into the resident cache
 * at row pos[m]: the projection half of _attn_decode (aneforge/llm.py:214-233) including the
 * masked positional cache write Kin*inv + k*oh, done here as one O(1) row store. */
int afx_qkv_rope_kv(int fmt, const void* w, const void* scale, const void* h, int ldh, const void* gamma,
                    float eps, int norm, const void* bias, int nq, int nk, int nv, int dh,
                    const void* cos_tab, const void* sin_tab, int rope, const int* pos, void* qout,
                    int ldq, void* kcache, void* vcache, long long kv_seq_stride,
                    long long kv_head_stride, int kv_len, int M, int K, int rows_hint, void* stream);

/* ---- codecs ----------------------------------------------------------------------------- */

/* GGUF Q4_0 blocks [N][K/32] (18 B) -> superblock layout (reference: GGUFView.get ->
 * gguf.quants.dequantize, aneforge/_gguf.py:34-39, which this keeps in 4-bit form). */
int afx_q4_0_repack(const void* blocks, void* qs, void* d, int N, int K, void* stream);
int afx_q4_0_unpack(const void* qs, const void* d, void* blocks, int N, int K, void* stream);
/* GGUF Q4_K super-blocks [N][K/256] (144 B: fp16 d, fp16 dmin, 12 B of 6-bit scales/mins, 128 B of
 * codes; reference: GGUFView.get -> gguf.quants.dequantize, aneforge/_gguf.py:34-39, kept 4-bit here)
 * -> codes qs [N][K/2] (the code bytes as they are) + hdr [N][K/256][5] u32 ({d | dmin << 16}, then
 * per sub-block pair p the bytes {sc(2p), sc(2p+1), m(2p), m(2p+1)}), the fmt 5 weight/scale pair. */
int afx_q4_k_repack(const void* blocks, void* qs, void* hdr, int N, int K, void* stream);
/* GGUF Q6_K super-blocks [N][K/256] (210 B: ql[128], qh[64], int8 scales[16], fp16 d; reference:
 * GGUFView.get -> gguf.quants.dequantize, aneforge/_gguf.py:34-39, kept 6-bit here) -> codes qs
 * [N][K/2] (per 32-weight chunk, byte j of dword k = low 4 bits of elements 8k+j | 8k+4+j << 4) +
 * sw [N][K/32][3] u32 (the chunk's high 2-bit parts, its two scales and d), the fmt 6 pair. */
int afx_q6_k_repack(const void* blocks, void* qs, void* sw, int N, int K, void* stream);
/* Dequantise through the GEMV's own unpack path into fp32 (bit-exact check of
 * quantize_per_row / Q4_0 / quantize_blockwise reconstruction, aneforge/_blob.py:20-25, 46-56). */
int afx_dequant(int fmt, const void* w, const void* scale, float* out, int N, int K, void* stream);
/* The same weights as fp16 rows out[n * ldo + k] (fmt 0 int8, 1 Q4_0, 3 blockwise, 4 int4, 5 Q4_K, 6 Q6_K): the fp16 values the
 * reference multiplies with -- for Q4_0 the fp16 cast of GGUFView.get (aneforge/_gguf.py:34-39).  The
 * batched prefill expands formats its GEMM does not read (Q4_0) into fp16 this way, one matrix at a time. */
int afx_dequant_f16(int fmt, const void* w, const void* scale, void* out, long long ldo, int N, int K,
                    void* stream);

/* ---- attention -------------------------------------------------------------------------- */

long long afx_decode_attn_ws_bytes(int B, int Hq, int Hkv, int D, int max_len, int nstep_hint);
/* Split-KV decode attention over an fp16 GQA cache: softmax(q K^T * scale (+mask)) V with
 * query head h reading kv head h / (Hq/Hkv).  Replaces af.sdpa at decode shape
 * (aneforge/graph.py:993-1040 -> aneforge/_compile.py:1442-1452 -> sdpa_fused,
 * aneforge/_bridges/ane_sdpa_fused.py:71-164) and the decomposed decode attention of
 * _attn_decode (aneforge/llm.py:234-236). */
int afx_decode_attn(const void* q, const void* k, const void* v, void* o, long long q_bs, long long q_hs,
                    long long kv_bs, long long kv_hs, int B, int Hq, int Hkv, int D, int ctx_len,
                    const int* pos, int max_len, const void* mask, long long mask_bs, int causal_off,
                    float scale, void* ws, long long ws_bytes, int nstep_hint, void* stream);
/* No counterpart in the reference.  afx_decode_attn without a workspace, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * the split partials go to a 32 MiB device array inside the library, one per device, held until the
 * process ends.  Calls whose partials (afx_decode_attn_ws_bytes) exceed 32 MiB fail with an error.
 * The stream must belong to the calling thread's current device.  Calls that overlap on one device
 * share the array and race. */
int afx_decode_attn_noalloc(const void* q, const void* k, const void* v, void* o, long long q_bs,
                            long long q_hs, long long kv_bs, long long kv_hs, int B, int Hq, int Hkv, int D,
                            int ctx_len, const int* pos, int max_len, const void* mask, long long mask_bs,
                            int causal_off, float scale, int nstep_hint, void* stream);

/* ---- norms, rope, sampling -------------------------------------------------------------- */

/* (aneforge/graph.py:293-301) */
int afx_rmsnorm(const void* x, int ldx, const void* gamma, float eps, void* y, int ldy, int M, int D,
                void* stream);
/* x*cos + rotate_half(x)*sin (aneforge/llm.py:96-105) */
int afx_rope(const void* x, void* y, int rows, int dh, const void* cos_tab, const void* sin_tab,
             const int* pos_dev, int pos0, int rows_per_pos, void* stream);
/* per-head RMSNorm then RoPE in place (QK-norm of _attn_decode, aneforge/llm.py:224-225, 227);
 * head h of row m at x + m*seq_stride + h*head_stride + pos_mul*pos[m] */
int afx_head_norm_rope(void* x, long long seq_stride, long long head_stride, int pos_mul, const int* pos,
                       int kv_len, int heads, int M, int dh, const void* gamma, float eps, const void* cos_tab,
                       const void* sin_tab, int rope, void* stream);
/* The next token of LlamaPrefill._sample (aneforge/llm.py:406-419) on the device: argmax (lowest
 * index) when temperature <= 0, else logits / T, the top-k logits (ties included), the top-p nucleus
 * (ties at its edge kept from the highest index down), and np.random.choice's draw: the first index
 * whose cumulative kept probability exceeds u.  params: device doubles {temperature, top_p, top_k};
 * u = uniforms[*step] (uniforms[0] when step is NULL).  The token goes to forced[*step] with
 * n_forced = *step + 1 (afx_decode_advance then takes it) and/or out[0].  ws: afx_sample_ws_bytes(V)
 * bytes, 8-byte aligned (the fp64 terms exp(x/T - max/T) and per-chunk sums and key histograms);
 * -1 for V outside [1, 2^21], which afx_sample rejects. */
long long afx_sample_ws_bytes(int V);
int afx_sample(const float* logits, int V, const double* params, const double* uniforms, const int* step,
               int* forced, int* n_forced, int* out, double* ws, long long ws_bytes, void* stream);
/* host embedding gather of LlamaPrefill.step (aneforge/llm.py:593-594), on the device */
int afx_embed(const void* table, const int* ids, void* out, int M, int D, int vocab, void* stream);
/* One step of the device-resident decode loop (aneforge/llm.py:584-627 step/_sample/generate):
 * token = forced[*step] while *step < *n_forced (prompt), else the greedy pick (lowest index on ties)
 * from the slots of afx_lm_head (or from the logits when slots is NULL); then hist[*step] = token,
 * ++*step, ++*pos, h = embed[token] (the host gather of :593-594).  With tie_margin (a device float),
 * the reference's near-tie rule (aneforge/llm.py:281, 395-404): when the two largest logits are closer
 * than margin * max|logit|, every logit inside that window of the largest is recomputed exactly from hn
 * (the head's fp16 input row [D]) and the head rows (head32 fp32 [V][D] if given, else head16), and
 * the largest exact value wins. */
int afx_decode_advance(const float* logits, const float* slots, int V, const float* tie_margin, const void* hn,
                       const void* head16, const float* head32, const int* forced, const int* n_forced, int* tok,
                       int* pos, int* hist, int hist_cap, int* step, const void* embed, void* h, int D, int vocab,
                       void* stream);
/* np.argmax per row (lowest index on ties) */
int afx_argmax(const float* x, int M, int V, int* out, void* stream);
/* graph-capturable fills (zeroing resident state, aneforge/llm.py:581-583) */
int afx_fill_i32(int* p, int n, int v, void* stream);
int afx_fill_f16(void* p, long long n, float v, void* stream);

/* ---- generic tensor ops for the af.compile executor (aneforge/graph.py op set) ---------- */

int afx_ew_binary(int op, const void* a, const long long* sa, const void* b, const long long* sb, void* y,
                  int rank, const int* dim, void* stream);
int afx_ew_select(const void* c, const long long* sc, const void* a, const long long* sa, const void* b,
                  const long long* sb, void* y, int rank, const int* dim, void* stream);
int afx_ew_unary(int op, const void* x, void* y, long long n, float alpha, float beta, void* stream);
int afx_copy_strided(const void* src, const long long* ss, void* dst, const long long* sd, int rank,
                     const int* dim, void* stream);
int afx_softmax(const void* x, void* y, int rows, int cols, void* stream);
int afx_reduce(int op, const void* x, void* y, int rows, int cols, void* stream);
int afx_bmm_f16(const void* A, const void* B, void* C, int batch, int M, int N, int K, long long sa,
                long long sb, long long sc, void* stream);

/* ---- mixture of experts (aneforge/moe.py:21-63) ----------------------------------------- */

/* softmax router -> top-k with the lowest-index fp16 tie rule (_topk_gate, moe.py:21-37) ->
 * optional renorm (moe.py:55-56) -> device bucketing of tokens per expert */
int afx_moe_topk(const float* logits, int T, int E, int k, int renorm, float* gate, int* sel, int* cnt,
                 int* list, void* stream);
/* active experts only: silu(x Wg_e^T) * (x Wu_e^T) (_experts_gate, moe.py:40-45, :57) */
int afx_moe_gateup(int fmt, const void* w, const void* scale, const void* x, int T, int k, int E, int F, int D,
                   const int* cnt, const int* list, void* act, int rows_hint, void* stream);
/* active experts only: act @ Wd_e (bmm_weight, moe.py:58).  ws (optional, may be NULL): an fp32
 * workspace; with up to 32 * T * k * D bytes, long expert rows are cut into up to 8 K slices, as for
 * afx_linear. */
int afx_moe_down(int fmt, const void* w, const void* scale, const void* act, int T, int k, int E, int F, int D,
                 const int* cnt, const int* list, float* y, int rows_hint, void* ws, long long ws_bytes,
                 void* stream);
/* The graph form of the top-k gate (_topk_gate, aneforge/moe.py:21-37): y = x on the k experts each
 * row of fp16 probabilities x [T][E] keeps (k rounds of the row maximum, the lowest index among exact
 * fp16 ties), 0 elsewhere; 1 <= k <= E <= 2049. */
int afx_topk_mask(const void* x, int T, int E, int k, void* y, void* stream);
/* h + sum_e gate * y_e (+ shared expert) (moe.py:59-63) */
int afx_moe_combine(const void* h, const float* y, const float* gate, const void* shared, void* out, int T,
                    int k, int D, void* stream);
/* The layer's routing for a decode batch in one launch: hn = RMSNorm(h) (the MLP norm before the
 * router, moe.py:40-63 via llm.py's block), logits = hn @ router^T, then afx_moe_topk's softmax,
 * top-k, renorm and bucketing (_topk_gate, moe.py:21-37, 55-56); bit for bit the outputs of
 * afx_rmsnorm + afx_linear (fp16 router, fp32 logits) + afx_moe_topk from T = 4 up (below 4 rows
 * afx_linear sums on its vector kernels, in another order; these logits are the MFMA ones).  T <= 16, E <= 16,
 * 256 <= D <= 4096 (D % 32 == 0), 16-byte aligned rows; logits (optional) [T][E] fp32.
 * sync (optional): afx_moe_route_sync_words() zeroed 32-bit words owned by the caller; with it the
 * router runs one workgroup per token (same outputs, bit for bit) and the last one buckets.  Calls
 * sharing one sync buffer must not overlap; without it, one workgroup does everything. */
int afx_moe_route(const void* h, int ldh, const void* gamma, float eps, const void* router, int T, int E, int D,
                  int k, int renorm, void* hn, int ldo, float* logits, float* gate, int* sel, int* cnt, int* list,
                  unsigned* sync, void* stream);
/* 32-bit words of afx_moe_route's sync buffer. */
int afx_moe_route_sync_words(void);
/* afx_moe_down followed by afx_moe_combine (bmm_weight and the gate-weighted sum, moe.py:58-63), with
 * the K-split's finishing sum folded into the combine: out is bit for bit that of the two calls. y
 * [T*k][D] fp32 scratch, ws as for afx_moe_down. */
int afx_moe_down_combine(int fmt, const void* w, const void* scale, const void* act, int T, int k, int E, int F,
                         int D, const int* cnt, const int* list, float* y, void* ws, long long ws_bytes,
                         const void* h, const float* gate, const void* shared, void* out, void* stream);

/* ---- batched prefill --------------------------------------------------------------------- */

/* Y = epilogue(X @ W^T) for M prompt rows on MFMA: the linears of the reference's batched
 * prefill (_prefiller, aneforge/llm.py:149-168, 489-544) with the compress="int8" weights of
 * aneforge/_compile.py:171-179 / 375-385 (fmt 0), fp16 (fmt 2) or compress="blockwise" (fmt 3,
 * 32-weight blocks, aneforge/_blob.py:46-56).  epi: 0 fp16, 1 fp16 +
 * residual, 2 fp32, 3 SwiGLU over interleaved gate/up rows (aneforge/llm.py:171-175). */
int afx_gemm(int fmt, const void* w, const void* scale, const void* x, int ldx, void* y, int ldy, int M, int N,
             int K, const void* bias, const void* residual, int epi, void* stream);
/* prompt [q | k | v] rows -> RoPE'd q and K/V cache rows at pos0.. (aneforge/llm.py:96-105, 149-168) */
int afx_qkv_split_rope(const void* qkv, int ldqkv, int M, int nq, int nk, int dh, const void* cos_tab,
                       const void* sin_tab, int pos0, int rope, void* q, int ldq, void* kcache, void* vcache,
                       long long kv_hs, int kv_len, void* stream);
/* causal GQA attention of the prompt over the resident cache (_attn_prefill_kv, aneforge/llm.py:149-168;
 * GQA as _repeat_kv3, :205-211; softmax as aneforge/_bridges/ane_sdpa_fused.py:57-68) */
int afx_prefill_attn(const void* q, int ldq, const void* kcache, const void* vcache, long long kv_hs, int Mmax,
                     void* o, int ldo, int M, int pos0, int Hq, int Hkv, int D, float scale, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* ANEFORGE_HIP_H */
