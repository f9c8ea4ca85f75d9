/*
 * od_mi355x.h — C ABI of the MI355X (gfx950) kernels for OpenDecider's quantized scoring forward path.
 *
 * Conventions (all entry points):
 *   - Pointers are DEVICE pointers of the current HIP device; bf16 tensors are passed as uint16_t bit patterns.
 *   - Sizes and strides are in ELEMENTS, int64_t; the last dimension of every tensor is contiguous.
 *   - `stream` is a hipStream_t passed as void* (NULL = the legacy default stream). Work is enqueued on it and
 *     the call returns without synchronizing.
 *   - Nothing allocates device or host memory and nothing synchronizes, so every call may be captured in a
 *     HIP graph. Calls on different streams may run concurrently when they share no output or workspace, with two
 *     exceptions that hold device-side state: od_branched_attn_split_noalloc (one static scratch array per GPU) and
 *     od_branched_attn_stream with splits (merge counters in its workspace); each says so below.
 *   - Return value: OD_OK (0) or a negative OD_ERR_* code; no exception crosses the ABI. od_strerror() gives
 *     the text. (The reference's own C ABI uses the same int-rc convention: deploy/llamacpp/od_llama.cpp:13-22,
 *     mapped to RuntimeError by src/opendecider/llamacpp.py:57-58.)
 */
#ifndef OD_MI355X_H
#define OD_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* od_stream_t;

#define OD_OK 0
#define OD_ERR_NULL (-1)        /* a required pointer is NULL */
#define OD_ERR_SHAPE (-2)       /* a size or stride is out of range or inconsistent */
#define OD_ERR_ALIGN (-3)       /* a pointer or leading dimension breaks the 16-byte alignment the kernel needs */
#define OD_ERR_UNSUPPORTED (-4) /* head dim / GQA ratio / row length outside what the kernels are built for */
#define OD_ERR_LAUNCH (-5)      /* the kernel launch failed (hipGetLastError) */
#define OD_ERR_SCRATCH (-6)     /* the work needs more than the library's static scratch (od_*_noalloc) */

/* How the branched attention turns the int8 state into K/V (the `dequant` argument). */
#define OD_DEQUANT_BF16 0 /* the reference's materialize: q.to(bf16) * s.to(bf16), one bf16 rounding per value */
#define OD_DEQUANT_FP32 1 /* the exact q * s (the K scale folded into the scores, V' rounded once to fp16) */

/* Text for an OD_* code. */
const char* od_strerror(int code);

/* ABI version of this library (bumped when a signature changes). */
int od_abi_version(void);

/*
 * od_act_quant — per-row dynamic int8 quantization, with optional SmoothQuant input scaling.
 * Replaces: Int8Tensor.quantize (src/opendecider/quant.py:36-41) applied per token to activations, the
 * SmoothedLinear input scaling x * inv_s (quant.py:325,328-329), and the dynamic activation quantizer inside
 * GemLite A8W8_int8_dynamic (called at quant.py:305-311, :336-347). Also used for Int8Linear's per-output-channel
 * weight quantization (quant.py:124-126), which is the same formula over weight rows.
 *   x      bf16 [M, K], row stride ldx
 *   inv_s  bf16 [K] or NULL; when given, each element is first rounded to bf16(x * inv_s)
 *   xq     int8 [M, K], row stride ldq (out)
 *   sx     fp32 [M] (out): scale = max(max_k |x|, 1e-8) / 127 (IEEE fp32 division)
 *   q = round_half_even(x / scale) (IEEE fp32 division), clamped to [-127, 127].
 * Bit-exact with the torch formula. Any M >= 0, K >= 1.
 */
int od_act_quant(const uint16_t* x, int64_t ldx, const uint16_t* inv_s, int8_t* xq, int64_t ldq, float* sx,
                 int64_t M, int64_t K, od_stream_t stream);

/*
 * od_gate_act_quant — od_act_quant of the attention output times the output gate.
 * Replaces: `o * torch.sigmoid(gate)` ahead of o_proj in the Qwen3.5 attention layer (src/opendecider/prefix_attn.py:
 * 84-85,130) fused with o_proj's input scaling and dynamic activation quantization (as od_act_quant).
 *   x     bf16 [M, K] (row stride ldx): the attention output;  gate  bf16 [M, K] (row stride ldg)
 *   each element first becomes bf16(x * bf16(sigmoid(g))) (sigmoid correctly rounded in fp32, then to bf16, as
 *   torch's bf16 sigmoid), then the od_act_quant formula (with inv_s when given). Other arguments as od_act_quant.
 */
int od_gate_act_quant(const uint16_t* x, int64_t ldx, const uint16_t* gate, int64_t ldg, const uint16_t* inv_s,
                      int8_t* xq, int64_t ldq, float* sx, int64_t M, int64_t K, od_stream_t stream);

/*
 * od_act_quant_f32 — the od_act_quant formula over fp32 rows.
 * Replaces: Int8Tensor.quantize (src/opendecider/quant.py:36-41) of float32 input, and of float16 / float64 input,
 * which the reference also quantizes from xf = x.float() (quant.py:38): the caller passes x.float().
 *   x   fp32 [M, K], row stride ldx;  xq int8 [M, K], row stride ldq (out);  sx fp32 [M] (out).
 * Same scale and bytes as the torch formula, NaN and inf rows included. Any M >= 0, K >= 1.
 */
int od_act_quant_f32(const float* x, int64_t ldx, int8_t* xq, int64_t ldq, float* sx, int64_t M, int64_t K,
                     od_stream_t stream);

/*
 * od_w8a8_gemm — int8 x int8 -> int32 GEMM on CDNA4 int8 MFMA with a bf16 dequant epilogue.
 * Replaces: the GEMM of GemLite A8W8_int8_dynamic behind gemlite_a8w8_ / smooth_a8w8_
 * (src/opendecider/quant.py:302-314, :332-350), and Int8Linear.forward's dequantize + F.linear
 * (quant.py:149-157) when attached through its `_fused` slot (quant.py:150-152, 398-409).
 *   a        int8 [M, K], row stride lda          sa  fp32 [M]  per-token activation scales
 *   w        int8 [N, K] (nn.Linear layout), ldw  sw  fp32 [N]  per-output-channel weight scales
 *   bias     bf16 [N] or NULL
 *   residual bf16 [M, N] (row stride ldr) or NULL, added in fp32 before the single rounding
 *   out      bf16 [M, N], row stride ldo, or NULL (then only acc is written)
 *   acc      int32 [M, N], row stride ldacc, or NULL (debug / parity: the exact accumulators)
 *   out = bf16( ((float(acc) * sa[m]) * sw[n]) + float(bias[n]) + float(residual[m, n]) )
 * Requires K % 16 == 0, lda/ldw % 16 == 0 and 16-byte aligned a/w (int8 rows are read in 16-byte chunks).
 */
int od_w8a8_gemm(const int8_t* a, int64_t lda, const float* sa, const int8_t* w, int64_t ldw, const float* sw,
                 const uint16_t* bias, const uint16_t* residual, int64_t ldr, uint16_t* out, int64_t ldo,
                 int32_t* acc, int64_t ldacc, int64_t M, int64_t N, int64_t K, od_stream_t stream);

/*
 * od_w8a8_gemm_swiglu — the gate+up projection of the decoder MLP with SwiGLU in its epilogue (no reference
 * counterpart as one function: the reference runs the two projections and silu(gate) * up as separate modules).
 *   w int8 [N, K] with N = 2F rows interleaved: row 2f is gate channel f, row 2f + 1 up channel f; sw fp32 [N].
 *   g = bf16(float(acc[m, 2f]) * sa[m] * sw[2f]), u likewise from row 2f + 1 (the od_w8a8_gemm output without bias
 *   or residual), out[m, f] = bf16(bf16(silu(g)) * u), out bf16 [M, F] with row stride ldo >= F: the values
 *   od_w8a8_gemm followed by od_silu_mul_quant's SwiGLU produce, without the [M, 2F] round trip through HBM.
 * Same requirements as od_w8a8_gemm; N must be even.
 */
int od_w8a8_gemm_swiglu(const int8_t* a, int64_t lda, const float* sa, const int8_t* w, int64_t ldw, const float* sw,
                        uint16_t* out, int64_t ldo, int64_t M, int64_t N, int64_t K, od_stream_t stream);

/*
 * od_w8a8_gemm_ws — od_w8a8_gemm's out (swiglu = 0) or od_w8a8_gemm_swiglu's (swiglu = 1: bias and residual NULL,
 * out bf16 [M, N/2]) with a caller workspace for split-K. Replaces the same reference calls as those two; the
 * workspace has no reference counterpart (GemLite picks its own split-K, quant.py:302-314).
 * Shapes with too few 256-row tiles to fill the chip (small M: the row and question passes) split K over several
 * workgroups per tile, each writing exact int32 partial sums to its plane of ws; a second pass adds the planes and
 * applies the same epilogue, so out is bit-identical to the unsplit call. ws: int32, 16-byte aligned, ws_ints
 * elements; od_w8a8_gemm_ws_size gives the size the current device's plan uses for (M, N, K) (0: no split). With
 * ws NULL or smaller than that, the call runs unsplit. Other requirements as od_w8a8_gemm.
 */
int od_w8a8_gemm_ws_size(int64_t M, int64_t N, int64_t K, int64_t* ws_ints);
int od_w8a8_gemm_ws(const int8_t* a, int64_t lda, const float* sa, const int8_t* w, int64_t ldw, const float* sw,
                    const uint16_t* bias, const uint16_t* residual, int64_t ldr, uint16_t* out, int64_t ldo, int64_t M,
                    int64_t N, int64_t K, int swiglu, int32_t* ws, int64_t ws_ints, od_stream_t stream);

/*
 * od_kv_quant_append — quantize new K or V rows (one scale per token per head) and append them to an int8 cache.
 * Replaces: maybe_quantize / Int8Tensor.quantize on cache tensors (quant.py:36-41,105-109) as called by
 * PackedCache.pack (src/opendecider/backbone.py:446) and by PrefixCache._take, which quantizes only the new
 * tokens' slice (src/opendecider/state_cache.py:79).
 *   x  bf16, logical shape [B, H, n_new, D], element strides (sxb, sxh, sxt), last dim contiguous
 *   q  int8 [B, H, cap, D] contiguous (out): rows n0 .. n0+n_new-1 are written
 *   s  fp32 [B, H, cap] contiguous (out): the matching scales
 * Same formula and bytes as od_act_quant per row; requires n0 + n_new <= cap.
 */
int od_kv_quant_append(const uint16_t* x, int64_t B, int64_t H, int64_t n_new, int64_t D, int64_t sxb, int64_t sxh,
                       int64_t sxt, int8_t* q, float* s, int64_t cap, int64_t n0, od_stream_t stream);

/*
 * od_kv_copy_rows — copy runs of int8 cache rows (with their fp32 scales) between two K/V buffers, every matrix and
 * head in one launch, bytes unchanged. Replaces: PrefixCache._take's copy of a snapshot's own tokens and
 * PrefixCache._restore's concatenation of the path's deltas followed by a re-pack (state_cache.py:68-93,106-124,
 * which dequantizes and quantizes again); here a restore writes the stored bytes back.
 *   src_q int8 / src_s fp32: n_mats matrices (a layer's K or V of one state) at element strides src_mat_q /
 *   src_mat_s, each [H][src_cap][D] / [H][src_cap]; dst likewise with dst_cap. seg: HOST array of n_seg runs
 *   (src_row, dst_row, n_rows), every run copied for every matrix and head. Requires D % 16 == 0, 16-byte aligned
 *   src_q / dst_q and matrix strides, each run inside both capacities (checked), n_mats * H <= 65535.
 */
int od_kv_copy_rows(const int8_t* src_q, const float* src_s, int64_t src_mat_q, int64_t src_mat_s, int64_t src_cap,
                    int8_t* dst_q, float* dst_s, int64_t dst_mat_q, int64_t dst_mat_s, int64_t dst_cap,
                    int64_t n_mats, int64_t H, int64_t D, const int64_t* seg, int64_t n_seg, od_stream_t stream);

/*
 * od_lm_head_logprob — log-prob of one token per row under an LM head whose rows are an int8 table, with the
 * normaliser over the whole vocabulary and no rows x vocabulary logits in memory. Replaces: Backbone.token_logprob
 * (src/opendecider/backbone.py:164-178) over Int8Embedding / Int8Linear rows (src/opendecider/quant.py:122-132,
 * 159-161,183-203), i.e. its chunk loop of dequant_rows + bf16 matmul + logsumexp + logaddexp and the fp32 target
 * term. Feeds the option-token LM feature (src/opendecider/v3.py:438-442,527-538).
 *   hb     bf16 [M, ldh]: bf16(h), the matmul operand
 *   hn     [M, ldhn], fp32 (hn_fp32 != 0) or bf16: h as the target term reads it (may alias hb when h is bf16)
 *   w      int8 [V, ldw] table rows; scale bf16 [V] (the per-row scale in the table's dtype)
 *   tok    int32 [M] device array: the token of each row (a token outside [0, V) gives NaN)
 *   out    fp32 [M] (out): sum_k float(h[m,k]) * float(w[tok,k] * scale[tok]) - logsumexp_v bf16(hb[m] . bf16(w[v] * scale[v]))
 *   ws     fp32 workspace of at least od_lm_head_logprob_ws(M, V) floats (per-row partial max / sum)
 * Requires K % 64 == 0, ldh % 8 == 0, ldw % 16 == 0, ldhn % 4 (fp32) or % 8 (bf16) == 0, hb, hn and w 16-byte
 * aligned, 256 * ldh * 2 and 256 * ldw below 2^31. Two launches (logit tiles with the partial log-sum-exp in
 * their epilogue, then a per-row combine).
 */
int od_lm_head_logprob_ws(int64_t M, int64_t V, int64_t* ws_floats);
int od_lm_head_logprob(const uint16_t* hb, int64_t ldh, const void* hn, int64_t ldhn, int hn_fp32, const int8_t* w,
                       int64_t ldw, const uint16_t* scale, const int32_t* tok, int64_t M, int64_t V, int64_t K,
                       float* out, float* ws, int64_t ws_floats, od_stream_t stream);

/*
 * od_lm_head_logprob_q4 — od_lm_head_logprob over a Q4_0 table (Q4Table, src/opendecider/quant.py:206-246): rows of
 * K / 32 blocks, each 16 bytes of nibbles (block positions 0-15 in the low nibbles, 16-31 in the high ones) and an
 * fp16 scale d; a value is (q - 8) * d. The logits use the reference's bf16 dequant_rows ((q - 8) in bf16 times
 * d.to(bf16), rounded to bf16); the target term uses (q - 8) * d in fp32.
 *   qs  uint8 [V, ldq >= K / 2] (ldq % 16 == 0, 16-byte aligned);  d  fp16 bits [V, ldd >= K / 32]
 * Other arguments, workspace and requirements as od_lm_head_logprob.
 */
int od_lm_head_logprob_q4(const uint16_t* hb, int64_t ldh, const void* hn, int64_t ldhn, int hn_fp32,
                          const uint8_t* qs, int64_t ldq, const uint16_t* d, int64_t ldd, const int32_t* tok,
                          int64_t M, int64_t V, int64_t K, float* out, float* ws, int64_t ws_floats,
                          od_stream_t stream);

/*
 * od_branched_attn — branched (Hydragen) option-row attention over an int8 shared state, one launch.
 * Replaces: _split_attention (src/opendecider/prefix_attn.py:43-76) with its two wide_attention launches
 * (src/opendecider/wide_attention.py:70-91) and the torch LSE merge (prefix_attn.py:74-76), the per-state loop
 * of _forward (prefix_attn.py:118-128), and the per-layer dequantized copy of the state K/V
 * (prefix_attn.py:145-149): the int8 state is read directly; every workgroup converts each 64-key block in its own
 * LDS, dequantized as `dequant` says: OD_DEQUANT_BF16, the reference's materialize (quant.py:45; keys and values
 * bf16(q * bf16(s)), one rounding each), or OD_DEQUANT_FP32, the exact q * s.
 *   q         bf16 [R, Hq, t, D], element strides (sqr, sqh, sqt)        R option rows of t tokens
 *   k_own     bf16 [R, Hkv, t, D], strides (skr, skh, skt)                each row's own keys (causal)
 *   v_own     bf16 [R, Hkv, t, D], strides (svr, svh, svt)
 *   kq, vq    int8 [Ns, Hkv, cap, D] contiguous                          the states' K/V (first T tokens used)
 *   ks, vs    fp32 [Ns, Hkv, cap] contiguous                             per-(token, head) scales
 *   kvalid    uint8 [Ns, T] (nonzero = real key) or NULL                  prefix key mask (pads / holes)
 *   row_start int32 [Ns + 1] device array: the rows of state s are rows row_start[s] .. row_start[s+1]-1
 *             (rows grouped by state; NULL means Ns == 1 and every row reads state 0)
 *   max_rows  the largest row_start[s+1] - row_start[s] (sizes the grid; must be exact or an upper bound)
 *   out       bf16 [R, Hq, t, D], strides (sor, soh, sot) (out)
 *   lse       fp32 [R, Hq, t] contiguous or NULL (out): natural-log LSE of the merged scaled scores
 *   dequant   OD_DEQUANT_BF16 or OD_DEQUANT_FP32 (else OD_ERR_UNSUPPORTED)
 * Query head h reads KV head h / (Hq / Hkv). Every query sees every valid prefix key and its own row's keys
 * 0..i (causal). A query with no visible key would return 0 (never happens: its own key is visible).
 * Supports D in {64, 128, 256} (the reference's dispatch set, prefix_attn.py:50; D = 256 runs one workgroup per CU),
 * Hq % Hkv == 0, t >= 1 (R * t * Hq / Hkv below 2^31), T <= cap.
 */
int od_branched_attn(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt,
                     const uint16_t* k_own, int64_t skr, int64_t skh, int64_t skt,
                     const uint16_t* v_own, int64_t svr, int64_t svh, int64_t svt,
                     const int8_t* kq, const float* ks, const int8_t* vq, const float* vs,
                     const uint8_t* kvalid, const int32_t* row_start, int64_t max_rows,
                     uint16_t* out, int64_t sor, int64_t soh, int64_t sot, float* lse,
                     int64_t R, int64_t Hq, int64_t Hkv, int64_t t, int64_t D, int64_t Ns, int64_t T, int64_t cap,
                     float scale, int dequant, od_stream_t stream);

/*
 * od_branched_attn_split — od_branched_attn with the state's keys split into nsplit contiguous ranges processed by
 * separate workgroups (for shapes with few slot tiles: few rows over a long state), merged by log-sum-exp.
 * Replaces: the same reference code as od_branched_attn; the split is an exact regrouping of the LSE merge of
 * prefix_attn.py:74-76 over more parts.
 *   nsplit     1 .. 256 (1 behaves as od_branched_attn and ignores ws)
 *   ws         fp32 workspace of at least ws_floats >= nsplit * R * Hq * t * (D + 1) floats, 16-byte aligned: each
 *              split's normalized partial output and LSE (caller-owned; contents undefined after the call)
 * Other arguments and the result as od_branched_attn. Two launches on `stream` (splits, then the merge).
 */
int od_branched_attn_split(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt,
                           const uint16_t* k_own, int64_t skr, int64_t skh, int64_t skt,
                           const uint16_t* v_own, int64_t svr, int64_t svh, int64_t svt,
                           const int8_t* kq, const float* ks, const int8_t* vq, const float* vs,
                           const uint8_t* kvalid, const int32_t* row_start, int64_t max_rows,
                           uint16_t* out, int64_t sor, int64_t soh, int64_t sot, float* lse,
                           int64_t R, int64_t Hq, int64_t Hkv, int64_t t, int64_t D, int64_t Ns, int64_t T,
                           int64_t cap, float scale, int dequant, int64_t nsplit, float* ws, int64_t ws_floats,
                           od_stream_t stream);

/*
 * od_branched_attn_stream — od_branched_attn_split for the few-slot case: every (state, KV head) carries at most 32
 * query slots (max_rows * t * Hq / Hkv <= 32, e.g. a yes/no decision of 2 options x 2 tokens over a long state), and
 * the attention is bound by reading the int8 state. One wave holds all slots of its (state, head) as one or two
 * 16-slot MFMA column tiles (one when max_rows * t * Hq / Hkv <= 16) and streams the int8 K/V from memory into
 * registers 32 keys at a time with non-temporal loads, dequantized there as `dequant` says (no block images, no LDS
 * staging); P enters the P.V product as two bf16 parts (hi + lo). Each slot's result depends on its own scores only
 * (option order cannot change it); results agree with od_branched_attn to the attention bar, not bit for bit.
 * Replaces: the same reference code as od_branched_attn (prefix_attn.py:43-76 with Kp/Vp materialized at :145-149).
 *   D          128 only (else OD_ERR_UNSUPPORTED); more than 32 slots per (state, head): OD_ERR_UNSUPPORTED
 *   max_rows   as od_branched_attn (an upper bound); a state whose row_start span holds more slots than the column
 *              tiles max_rows sized (16 or 32) gets NaN outputs and LSEs instead of an attention result
 *   nsplit     1 .. 256: the keys of a (state, head) split over nsplit workgroups of 8 waves. A CU runs one such
 *              workgroup at a time: Ns * Hkv * nsplit at (or just below) a multiple of the CU count fills the GPU
 *              without a partial last round (4 splits for 64 (state, head) pairs on MI355X's 256 CUs)
 *   ws         nsplit > 1: fp32 workspace of ws_floats >= nsplit * R * Hq * t * (D + 1) + Ns * Hkv floats, 16-byte
 *              aligned: the splits' normalized partials and LSEs, then one int32 merge counter per (state, KV head).
 *              The counters must be zero when the call starts and are zero again when it ends (the last split of a
 *              (state, head) to finish merges the partials and resets its counter), so a workspace zeroed once serves
 *              every later call; calls that share a workspace must not overlap
 * Other arguments and the result as od_branched_attn_split. One launch (the split merge is fused into it).
 */
int od_branched_attn_stream(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt,
                            const uint16_t* k_own, int64_t skr, int64_t skh, int64_t skt,
                            const uint16_t* v_own, int64_t svr, int64_t svh, int64_t svt,
                            const int8_t* kq, const float* ks, const int8_t* vq, const float* vs,
                            const uint8_t* kvalid, const int32_t* row_start, int64_t max_rows,
                            uint16_t* out, int64_t sor, int64_t soh, int64_t sot, float* lse,
                            int64_t R, int64_t Hq, int64_t Hkv, int64_t t, int64_t D, int64_t Ns, int64_t T,
                            int64_t cap, float scale, int dequant, int64_t nsplit, float* ws, int64_t ws_floats,
                            od_stream_t stream);

/*
 * od_branched_attn_split_noalloc — od_branched_attn_split without a workspace argument and without any allocation:
 * the per-split partials go to a static device array inside the library (OD_SPLIT_SCRATCH_FLOATS floats = 64 MiB per
 * GPU). The array is part of the library's code object, so every GPU the library is loaded on holds it from then
 * until the process ends, whether or not this entry point is ever called. No counterpart in the reference: it is
 * for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 *   arguments, result and launches as od_branched_attn_split (without ws / ws_floats)
 *   nsplit * R * Hq * t * (D + 1) must not exceed OD_SPLIT_SCRATCH_FLOATS (else OD_ERR_SCRATCH, nothing launched);
 *   nsplit = 1 uses no scratch.
 * Every call on one GPU shares that GPU's array, which keeps the last call's partials (every partial a call's merge
 * reads is written by the same call, so nothing needs clearing): calls that overlap on one GPU (two streams, two
 * threads) race and must be serialized by the caller.
 */
#define OD_SPLIT_SCRATCH_FLOATS (16ll * 1024 * 1024)
int od_branched_attn_split_noalloc(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt,
                                   const uint16_t* k_own, int64_t skr, int64_t skh, int64_t skt,
                                   const uint16_t* v_own, int64_t svr, int64_t svh, int64_t svt,
                                   const int8_t* kq, const float* ks, const int8_t* vq, const float* vs,
                                   const uint8_t* kvalid, const int32_t* row_start, int64_t max_rows,
                                   uint16_t* out, int64_t sor, int64_t soh, int64_t sot, float* lse,
                                   int64_t R, int64_t Hq, int64_t Hkv, int64_t t, int64_t D, int64_t Ns, int64_t T,
                                   int64_t cap, float scale, int dequant, int64_t nsplit, od_stream_t stream);

/*
 * od_attn_stage_size — bytes of the block images od_attn_stage writes for a state of Ns x Hkv heads and T keys:
 * Ns * Hkv * ceil(T / 64) images of 4 * 64 * D + 528 bytes. No GPU work.
 * Has no counterpart in the reference (a size query for od_attn_stage's output buffer).
 */
int od_attn_stage_size(int64_t Ns, int64_t Hkv, int64_t T, int64_t D, int64_t* img_bytes);

/*
 * od_attn_stage — converts an int8 state into attention block images, once for all the workgroups that read it.
 * Replaces: the per-layer dequantized copy of the state K/V (prefix_attn.py:145-149, quant.py:40-47
 * materialize), in the form od_branched_attn_staged consumes: per (state, head, 64-key block) the keys in bf16
 * with their fp32 score multipliers, the values in fp16 times a power of two, both swizzled for the LDS fragment
 * reads, a -inf row for masked keys and the block's V exponent. With OD_DEQUANT_BF16 the keys and values are the
 * reference's materialized bf16(q * bf16(s)) and the multiplier is the softmax scale; with OD_DEQUANT_FP32 the keys
 * are the int8 values, the multiplier is the K scale times the softmax scale, and the values are fp16(q * s).
 *   kq, vq, ks, vs, kvalid, Ns, Hkv, T, cap, D, dequant   as od_branched_attn
 *   scale      the softmax scale of the attention calls that will read the images
 *   img        device buffer of at least od_attn_stage_size bytes, 16-byte aligned (out)
 * One launch on `stream`. The images equal what od_branched_attn builds in LDS, so od_branched_attn_staged over
 * them returns the same bits as od_branched_attn.
 */
int od_attn_stage(const int8_t* kq, const float* ks, const int8_t* vq, const float* vs, const uint8_t* kvalid,
                  int64_t Ns, int64_t Hkv, int64_t T, int64_t cap, int64_t D, float scale, int dequant,
                  void* img, int64_t img_bytes, od_stream_t stream);

/*
 * od_attn_stage_bf16 — block images of a DENSE bf16 state, for od_branched_attn_staged.
 * Replaces: the prefix part of _split_attention when its caller passes materialized bf16 K/V
 * (src/opendecider/prefix_attn.py:43-57, called at :127 with K/V from :145-149), i.e. the reference's
 * wide_attention prefix call (wide_attention.py:70-91) and its LSE merge with the own part (prefix_attn.py:74-76):
 * the images feed the same one-softmax attention as the int8 state's.
 *   k, v      bf16 [Ns, Hkv, T, D] at element strides (skb, skh, skt) / (svb, svh, svt) (multiples of 8), last dim
 *             contiguous, 16-byte aligned
 *   kvalid    uint8 [Ns, T] or NULL (as od_branched_attn)
 *   scale     the softmax scale of the attention calls that will read the images
 *   img       device buffer of at least od_attn_stage_size bytes, 16-byte aligned (out)
 * Keys are used as they are; values become fp16(v 2^-eb) with 2^eb above the block's largest |v| (exact down to
 * 2^(eb - 14)). D in {64, 128, 256}. One launch on `stream`.
 */
int od_attn_stage_bf16(const uint16_t* k, int64_t skb, int64_t skh, int64_t skt, const uint16_t* v, int64_t svb,
                       int64_t svh, int64_t svt, const uint8_t* kvalid, int64_t Ns, int64_t Hkv, int64_t T, int64_t D,
                       float scale, void* img, int64_t img_bytes, od_stream_t stream);

/*
 * od_branched_attn_staged — od_branched_attn_split over block images from od_attn_stage / od_attn_stage_bf16: each workgroup copies the
 * images straight into LDS (global_load_lds) instead of converting the int8 state itself.
 * Replaces: the same reference code as od_branched_attn.
 *   img, img_bytes   the images of the state (Ns, Hkv, T, D and scale as passed to od_attn_stage; the images carry
 *                    the dequantization)
 *   nsplit, ws, ws_floats   as od_branched_attn_split (nsplit = 1 ignores ws)
 * Other arguments and the result as od_branched_attn.
 */
int od_branched_attn_staged(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt,
                            const uint16_t* k_own, int64_t skr, int64_t skh, int64_t skt,
                            const uint16_t* v_own, int64_t svr, int64_t svh, int64_t svt,
                            const void* img, int64_t img_bytes, const int32_t* row_start, int64_t max_rows,
                            uint16_t* out, int64_t sor, int64_t soh, int64_t sot, float* lse,
                            int64_t R, int64_t Hq, int64_t Hkv, int64_t t, int64_t D, int64_t Ns, int64_t T,
                            float scale, int64_t nsplit, float* ws, int64_t ws_floats, od_stream_t stream);

/*
 * od_branched_attn_staged2 — the branched attention over a TWO-LEVEL shared prefix: every row group (a question)
 * attends the blocks of its state, then the blocks of its own question K/V, then each row's own tokens causally, in
 * one online softmax. Replaces: the question-cache path of the attention layer, which joins the state K/V and each
 * question's own K/V along the keys before the split attention (src/opendecider/prefix_attn.py:94-99, driven by
 * v3.py:446-534 _branched_feats_qcache) and the per-question LSE merge with the own part (prefix_attn.py:74-76).
 *   img, img_bytes   level 1: block images of n_states states x Hkv heads x T keys (od_attn_stage, int8 state)
 *   group_state      int32 [n_groups] device array: the state of each row group (NULL: group g reads state g); a
 *                    value outside [0, n_states) reads no level-1 keys
 *   img2, img2_bytes level 2: block images of n_groups x Hkv heads x T2 keys (od_attn_stage_bf16 of the questions'
 *                    dense bf16 K/V, pads masked with its kvalid); T2 = 0: no second level
 *   row_start        int32 [n_groups + 1]: the rows of group g (NULL: n_groups == 1)
 *   other arguments, workspace and result as od_branched_attn_staged
 */
int od_branched_attn_staged2(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt,
                             const uint16_t* k_own, int64_t skr, int64_t skh, int64_t skt,
                             const uint16_t* v_own, int64_t svr, int64_t svh, int64_t svt,
                             const void* img, int64_t img_bytes, const int32_t* group_state, int64_t n_states,
                             int64_t T, const void* img2, int64_t img2_bytes, int64_t T2, const int32_t* row_start,
                             int64_t max_rows, uint16_t* out, int64_t sor, int64_t soh, int64_t sot, float* lse,
                             int64_t R, int64_t Hq, int64_t Hkv, int64_t t, int64_t D, int64_t n_groups, float scale,
                             int64_t nsplit, float* ws, int64_t ws_floats, od_stream_t stream);

/*
 * od_wide_attn — flash attention over bf16 K/V.
 * Replaces: wide_attention / _wide_fwd (src/opendecider/wide_attention.py:13-91).
 *   q      bf16 [B, H, T, DK], element strides (sqb, sqh, sqt)
 *   k      bf16 [B, G, S, DK], strides (skb, skg, sks)
 *   v      bf16 [B, G, S, DV], strides (svb, svg, svs)
 *   kvalid uint8 [B, S] with row stride smb (nonzero = real key) or NULL
 *   out    bf16 [B, H, T, DV], strides (sob, soh, sot) (out)
 *   lse    fp32 [B, H, T] contiguous or NULL (out): natural-log log-sum-exp of the scaled scores, -inf where a
 *          query sees no key
 * Query head h reads KV group h / (H / G); queries are the last T of the S key positions (query t sits at t + S - T
 * and, with causal != 0, sees keys 0 .. t + S - T). A query with no visible key returns 0. P is rounded to bf16
 * before the P.V product, as in the reference. Supports H % G == 0, DK <= 512 with DK % 8 == 0, DV in
 * {64, 128, 256}; element strides multiples of 8 (q, k, v) and 4 (out); q, k, v 16-byte aligned, out 8-byte; a
 * positive finite scale (else OD_ERR_UNSUPPORTED: the block max is taken on the unscaled scores).
 */
int od_wide_attn(const uint16_t* q, int64_t sqb, int64_t sqh, int64_t sqt, const uint16_t* k, int64_t skb,
                 int64_t skg, int64_t sks, const uint16_t* v, int64_t svb, int64_t svg, int64_t svs,
                 const uint8_t* kvalid, int64_t smb, uint16_t* out, int64_t sob, int64_t soh, int64_t sot, float* lse,
                 int64_t B, int64_t H, int64_t G, int64_t T, int64_t S, int64_t DK, int64_t DV, int causal,
                 float scale, od_stream_t stream);

/*
 * Row kernels of the dense decoder layer that carries the path in the decision-forward harness (not reference
 * functions: the reference runs these steps inside HF Qwen3.5 modules; they are fused here around the W8A8 GEMMs).
 *
 * od_rmsnorm_quant: y = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))), optionally y = bf16(y * inv_s), then the
 *   od_act_quant formula per row. x bf16 [M, K] (row stride ldx), w / inv_s bf16 [K], xq int8 [M, ldq], sx fp32 [M].
 */
int od_rmsnorm_quant(const uint16_t* x, int64_t ldx, const uint16_t* w, const uint16_t* inv_s, float eps, int8_t* xq,
                     int64_t ldq, float* sx, int64_t M, int64_t K, od_stream_t stream);

/*
 * od_rmsnorm_quant_ex: od_rmsnorm_quant with the weight convention chosen by weight_offset: 0 is the one above;
 *   1 is Qwen3.5's zero-centred norm (transformers' Qwen3_5RMSNorm, the input / post-attention / final norms of the
 *   reference's default backbone, configs/backbone.yaml:1-4): y = bf16((x * r) * (1 + w)), products and the sum
 *   1 + w in fp32, one rounding. Any other weight_offset returns OD_ERR_UNSUPPORTED.
 */
int od_rmsnorm_quant_ex(const uint16_t* x, int64_t ldx, const uint16_t* w, const uint16_t* inv_s, float eps,
                        int weight_offset, int8_t* xq, int64_t ldq, float* sx, int64_t M, int64_t K,
                        od_stream_t stream);

/*
 * od_silu_mul_quant: y = bf16(bf16(silu(g)) * u) with g = gu[:, :F], u = gu[:, F:2F] (fused gate+up GEMM output,
 *   row stride ldg), optionally y = bf16(y * inv_s), then the od_act_quant formula per row -> aq int8 [M, ldq],
 *   sa fp32 [M].
 */
int od_silu_mul_quant(const uint16_t* gu, int64_t ldg, int64_t F, const uint16_t* inv_s, int8_t* aq, int64_t ldq,
                      float* sa, int64_t M, od_stream_t stream);

/*
 * od_qk_norm_rope: in place on the QKV GEMM output qkv bf16 [M, ld] whose row holds n_heads_q query heads then
 *   n_heads_k key heads of D values: per head n = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))) (w = q_w or k_w,
 *   bf16 [D]), then rotary embedding out = bf16(bf16(n * cos) + bf16(rotate_half(n) * sin)) with cos/sin bf16
 *   tables [n_pos, D/2] indexed by pos[row] (int32 [M]; a position outside [0, n_pos) yields NaN). Same convention
 *   as the reference's apply_rotary_pos_emb call (src/opendecider/prefix_attn.py:81,90). D in {64, 128}.
 */
int od_qk_norm_rope(uint16_t* qkv, int64_t ld, int64_t M, int64_t n_heads_q, int64_t n_heads_k, int64_t D,
                    const uint16_t* q_w, const uint16_t* k_w, const uint16_t* cos_t, const uint16_t* sin_t,
                    int64_t n_pos, const int32_t* pos, float eps, od_stream_t stream);

/*
 * od_qk_norm_rope_ex: od_qk_norm_rope for Qwen3.5's full-attention heads as well: D in {64, 128, 256}; rot_dim = D
 *   (full rotary) or D / 4 (partial rotary, Qwen3.5's partial_rotary_factor 0.25: rotate_half acts on dims
 *   0 .. rot_dim - 1, pairs (d, d + rot_dim / 2), and dims rot_dim .. D - 1 keep their normalized values, as
 *   transformers' apply_rotary_pos_emb does for a cos/sin table narrower than the head); the tables are
 *   [n_pos, rot_dim / 2]. weight_offset as od_rmsnorm_quant_ex (1: the q/k norms are Qwen3_5RMSNorm,
 *   n = bf16((x * r) * (1 + w))). Needs ld % 4 == 0 and 8-byte aligned qkv / weights / tables (else OD_ERR_ALIGN)
 *   except for the D in {64, 128}, full-rotary, weight_offset 0 case, which od_qk_norm_rope also serves unaligned.
 */
int od_qk_norm_rope_ex(uint16_t* qkv, int64_t ld, int64_t M, int64_t n_heads_q, int64_t n_heads_k, int64_t D,
                       int64_t rot_dim, int weight_offset, const uint16_t* q_w, const uint16_t* k_w,
                       const uint16_t* cos_t, const uint16_t* sin_t, int64_t n_pos, const int32_t* pos, float eps,
                       od_stream_t stream);

/*
 * od_qk_norm_rope_kv_append: od_qk_norm_rope plus the int8 K/V append of the same tokens, in one pass over the QKV
 *   GEMM output. Replaces, for a state prefill: the q/k norm + RoPE of the attention layer (prefix_attn.py:81-90)
 *   followed by the quantization of the new tokens' K/V slice that PrefixCache._take (state_cache.py:79) and
 *   PackedCache.pack (backbone.py:446) run through Int8Tensor.quantize (quant.py:36-41).
 *   qkv bf16 [B * S, ld], row b * S + i = token i of state b, holding n_heads_q query heads, n_heads_k key heads
 *   and n_heads_k value heads of D values. Query and key heads are normalized and rotated in place as in
 *   od_qk_norm_rope (pos int32 [B * S]); then every key head (after RoPE) and value head is quantized per (token,
 *   head) into kq / vq int8 [B, n_heads_k, cap, D] rows n0 .. n0 + S - 1 with scales ks / vs fp32 [B, n_heads_k, cap]:
 *   the bytes od_kv_quant_append writes for the same bf16 values. Requires n0 + S <= cap, D in {64, 128},
 *   ld % 4 == 0, 8-byte aligned qkv / weights / tables and 4-byte aligned kq / vq (else OD_ERR_ALIGN).
 */
int od_qk_norm_rope_kv_append(uint16_t* qkv, int64_t ld, int64_t B, int64_t S, int64_t n_heads_q, int64_t n_heads_k,
                              int64_t D, const uint16_t* q_w, const uint16_t* k_w, const uint16_t* cos_t,
                              const uint16_t* sin_t, int64_t n_pos, const int32_t* pos, float eps, int8_t* kq,
                              float* ks, int8_t* vq, float* vs, int64_t cap, int64_t n0, od_stream_t stream);

/*
 * od_qk_norm_rope_kv_append_ex: od_qk_norm_rope_kv_append with od_qk_norm_rope_ex's head dims (64, 128, 256),
 *   rot_dim (D or D / 4) and weight_offset (0 or 1); the same alignment requirements.
 */
int od_qk_norm_rope_kv_append_ex(uint16_t* qkv, int64_t ld, int64_t B, int64_t S, int64_t n_heads_q,
                                 int64_t n_heads_k, int64_t D, int64_t rot_dim, int weight_offset,
                                 const uint16_t* q_w, const uint16_t* k_w, const uint16_t* cos_t,
                                 const uint16_t* sin_t, int64_t n_pos, const int32_t* pos, float eps, int8_t* kq,
                                 float* ks, int8_t* vq, float* vs, int64_t cap, int64_t n0, od_stream_t stream);

/*
 * Gated DeltaNet (linear-attention) layers of the Qwen3.5 hybrid backbone: the passes between the layer's input
 * projection (one W8A8 GEMM giving [qkv | z | b | a]) and its out_proj. Replaces the body of transformers'
 * Qwen3_5GatedDeltaNet.forward that the reference runs (src/opendecider/backbone.py:256-289 padded continuations,
 * src/opendecider/skipkv.py:208-231): causal_conv1d_fn / causal_conv1d_update + SiLU, l2norm, the gates, the
 * chunked / recurrent gated delta rule and Qwen3_5RMSNormGated; for option rows continuing a shared state, the
 * per-row state copies of the reference (backbone.py:529-571 row_states) become reads of the one shared state
 * (docs/branched_shared_prefix_math.md:16-37).
 * Token layout: M = S * L tokens, sequence s = tokens s L .. s L + L - 1. Dims: n_k key heads of dk, n_v value heads
 * of dv (n_v % n_k == 0, value head h reads key head h / (n_v / n_k)), C = 2 n_k dk + n_v dv conv channels.
 *
 * od_gdn_prep: proj bf16 [M, ldp] ([qkv C | z n_v dv | b n_v | a n_v], ldp % 8 == 0, 16-byte aligned); conv_w bf16
 *   [C, 4]; conv_in bf16 [n_states, 3, C] (the previous 3 pre-conv inputs of each state) or NULL (zeros); seq_state
 *   int32 [S] (the state sequence s continues; NULL: state s; an index outside [0, n_states) reads zeros); A_log,
 *   dt_bias bf16 [n_v]. Writes qk bf16 [M, 2 n_k dk] (l2-normed q heads then k heads), v bf16 [M, n_v dv], g fp32
 *   [M, n_v] = -exp(A_log) softplus(a + dt_bias), beta fp32 [M, n_v] = bf16(sigmoid(b)), and, if conv_out is not NULL,
 *   bf16 [S, 3, C]: the last 3 pre-conv inputs of each [state ; sequence] (conv_out must not overlap conv_in).
 *   dk, dv multiples of 16 with dk / 16 a power of two <= 64, C <= 16384, n_v <= C / 16.
 * od_gdn_recurrence: qk, v, g, beta as od_gdn_prep writes them; init fp32 [n_states, n_v, dk, dv] or NULL (zeros),
 *   read through seq_state as above; writes o bf16 [M, n_v dv] and, if final_state is not NULL, fp32 [S, n_v, dk,
 *   dv] (final_state may alias init only when seq_state is NULL). dk == 128, dv % 32 == 0; L >= 1.
 * od_gdn_recurrence_chunked: the same inputs, outputs and rules as od_gdn_recurrence, computed in chunks of 32 tokens
 *   on bf16 MFMA (the WY form of the chunked delta rule, as torch_chunk_gated_delta_rule evaluates it; fp32 operands
 *   split into bf16 hi + lo, fp32 accumulation): two launches, the first writing per-chunk matrices into the
 *   caller's workspace ws (ws_floats >= what od_gdn_chunk_ws_size gives, 16-byte aligned), the second reading them
 *   (the workspace must not be shared by calls that overlap). dv % 64 == 0.
 * od_gdn_norm_quant: o bf16 [M, ldo], z bf16 [M, ldz] (the z columns of proj), w bf16 [dv], inv_s bf16 [n_v dv] or
 *   NULL: y = bf16(bf16(w * bf16(o * r)) * silu(z)) per value head (r = 1 / sqrt(mean(o^2) + eps)), then
 *   od_act_quant's bytes and scale of y (times inv_s): xq int8 [M, ldq] (ldq % 16 == 0), sx fp32 [M].
 */
int od_gdn_prep(const uint16_t* proj, int64_t ldp, const uint16_t* conv_w, const uint16_t* conv_in,
                const int32_t* seq_state, int64_t n_states, const uint16_t* A_log, const uint16_t* dt_bias, int64_t S,
                int64_t L, int64_t n_k, int64_t n_v, int64_t dk, int64_t dv, uint16_t* qk, uint16_t* v, float* g,
                float* beta, uint16_t* conv_out, od_stream_t stream);
/*
 * od_gdn_prep_ex: od_gdn_prep for right-padded sequences, the reference's Backbone.padded_continuation
 *   (src/opendecider/backbone.py:256-289, used by the batched question pass, v3.py:446-497): seq_len int32 [S] holds
 *   each sequence's real tokens (NULL: all L; values are clamped into [0, L]). A pad token gets beta = 0 and g = -0,
 *   what the reference's b = a = -inf give, so the recurrence carries the state through it unchanged; conv_out takes
 *   the 3 pre-conv inputs of [state ; sequence] that end at the last real token (the state's own window when
 *   seq_len is 0). Outputs at pad positions are computed from the pad tokens and carry no meaning.
 */
int od_gdn_prep_ex(const uint16_t* proj, int64_t ldp, const uint16_t* conv_w, const uint16_t* conv_in,
                   const int32_t* seq_state, int64_t n_states, const int32_t* seq_len, const uint16_t* A_log,
                   const uint16_t* dt_bias, int64_t S, int64_t L, int64_t n_k, int64_t n_v, int64_t dk, int64_t dv,
                   uint16_t* qk, uint16_t* v, float* g, float* beta, uint16_t* conv_out, od_stream_t stream);
int od_gdn_recurrence(const uint16_t* qk, const uint16_t* v, const float* g, const float* beta, const float* init,
                      const int32_t* seq_state, int64_t n_states, int64_t S, int64_t L, int64_t n_k, int64_t n_v,
                      int64_t dk, int64_t dv, uint16_t* o, float* final_state, od_stream_t stream);
int od_gdn_chunk_ws_size(int64_t S, int64_t L, int64_t n_v, int64_t* ws_floats);
int od_gdn_recurrence_chunked(const uint16_t* qk, const uint16_t* v, const float* g, const float* beta,
                              const float* init, const int32_t* seq_state, int64_t n_states, int64_t S, int64_t L,
                              int64_t n_k, int64_t n_v, int64_t dk, int64_t dv, uint16_t* o, float* final_state,
                              float* ws, int64_t ws_floats, od_stream_t stream);
int od_gdn_norm_quant(const uint16_t* o, int64_t ldo, const uint16_t* z, int64_t ldz, const uint16_t* w,
                      const uint16_t* inv_s, float eps, int64_t M, int64_t n_v, int64_t dv, int8_t* xq, int64_t ldq,
                      float* sx, od_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* OD_MI355X_H */
