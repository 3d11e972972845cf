/* dj.h — the C ABI of the MI355X (gfx950) scoring path of decision.js.
 *
 * It replaces the WebGPU layer of the reference: src/gpu.ts (device, weight upload, tiled weights,
 * recorder, profiling) and the WGSL kernels of src/kernels.ts, src/d3-kernels.ts, src/eg2-kernels.ts and
 * src/encoder-kernels.ts. The engines (host packing + dispatch order) stay on the host side and call this
 * library; every pointer called `dev` below is device memory from dj_buf_alloc, every `host` pointer is
 * ordinary host memory. No type from PyTorch or any other framework appears here.
 *
 * Conventions
 *  - Every function returns DJ_OK (0) or a nonzero DJ_E* status; dj_last_error() then holds a message
 *    ("decision.js: ..."), thread-local, like the reference's thrown Error (gpu.ts:260, d1.ts:68).
 *  - Activations are IEEE binary16 stored as uint16_t; reductions run in f32 (kernels.ts:1).
 *  - Ops take a recorder (dj_rec): they are queued on the context's HIP stream in call order and run when
 *    dj_rec_finish() is called, as the reference records one command buffer per forward (gpu.ts:176-281).
 *  - One forward at a time per context (the reference's D1.queue, d1.ts:112-119). Not thread-safe.
 */
#ifndef DJ_H
#define DJ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DJ_ABI_VERSION 1

enum {
  DJ_OK = 0,
  DJ_EINVAL = 1,    /* bad argument (shape, null pointer, unsupported combination) */
  DJ_EHIP = 2,      /* the HIP runtime reported an error */
  DJ_ENOMEM = 3,    /* device or host allocation failed */
  DJ_ESTATE = 4,    /* call out of order (e.g. an op outside a recorder) */
  DJ_EINJECT = 5,   /* an error forced by DJ_FAULT_INJECT=<op>[:<n>] (tests of the host's error path: the op
                       fails before launching, every time or its next n times; read by dj_init) */
};

typedef struct dj_ctx dj_ctx;
typedef struct dj_rec dj_rec;
typedef struct dj_weight dj_weight;

/* ---------------------------------------------------------------- errors, version */

/* The message of the last failed call on this thread ("" if none).
 * Replaces: the thrown `Error("decision.js: ...")` of gpu.ts:66, 78, 260 and d1.ts:68. */
const char *dj_last_error(void);
int dj_abi_version(void);

/* ---------------------------------------------------------------- device (gpu.ts:38-54) */

/* Opens HIP device `ordinal` with one stream of default priority.
 * Replaces: requestDevice() (gpu.ts:38-54) and `new GpuEngine(device, ...)` (gpu.ts:101-105). */
int dj_init(int ordinal, dj_ctx **out);
/* Frees everything the context still owns (buffers, weights, cached graphs).
 * Replaces: GpuEngine.destroy (gpu.ts:108-110) / D1.destroy (d1.ts:108-110). */
int dj_destroy(dj_ctx *ctx);
/* Device name (gcnArchName), compute units and total memory; `name` gets at most `cap` bytes. */
int dj_device_info(dj_ctx *ctx, char *name, size_t cap, int *compute_units, size_t *total_mem);

/* ---------------------------------------------------------------- buffers (gpu.ts:148-174, 235-267) */

/* Device buffer of `bytes` (rounded up to 256). Replaces storage()/activations()/activationRows(). */
int dj_buf_alloc(dj_ctx *ctx, size_t bytes, void **dev);
int dj_buf_free(dj_ctx *ctx, void *dev);
/* Synchronous copies between host and device memory (load-time uploads: queue.writeBuffer, gpu.ts:69). */
int dj_buf_write(dj_ctx *ctx, void *dev, const void *host, size_t bytes);
int dj_buf_read(dj_ctx *ctx, void *host, const void *dev, size_t bytes);

/* ---------------------------------------------------------------- weights (gpu.ts:6-11, 57-88, 114-133) */

enum {
  DJ_W_PLAIN = 0,   /* kept in the file's layout: rows gathered (GATHER_Q8/Q4) and read as LM head (LEAF_LOGITS) */
  DJ_W_MFMA = 1,    /* repacked for the q8/q4 block-dequant MFMA GEMM (dj_matmul) */
  DJ_W_MFMA_GLU = 2, /* as DJ_W_MFMA for a fused [w1; w3] (N = 2I), 16-column blocks of w1 and w3 interleaved
                        so one output tile holds a gate column and its up column (dj_matmul_glu) */
  DJ_W_DIRECT = 16   /* flag on DJ_W_MFMA / DJ_W_MFMA_GLU: dequantize once at load into f16 MFMA blocks (the
                        reference's directWeights option, gpu.ts:16-20, 114-133): bit-identical f16 weights,
                        2 bytes per weight, no dequantization in the GEMM */
};

/* A quantized weight [N, K] from the weights.bin encodings of export_common.py:4-7, 64-97:
 *   bits 8: codes u8 [N, K] (code = q + 128), scales f16 [N, K/32]
 *   bits 4: codes u8 [N, K/2] (two codes per byte, low nibble first, code = q + 8), scales f16 [N, K/32]
 * `codes`/`scales` are host pointers; the device copy is repacked per `layout` and owned by the context.
 * Replaces: loadWeights' per-tensor upload (gpu.ts:63-85) and tileWeights (gpu.ts:114-133,
 * kernels.ts:522-543), keeping the weights quantized. K % 32 == 0; N % 16 == 0 and K % 64 == 0 for MFMA. */
int dj_weight_q(dj_ctx *ctx, const void *codes, const void *scales, int N, int K, int bits, int layout,
                dj_weight **out);
int dj_weight_free(dj_ctx *ctx, dj_weight *w);
/* Device bytes the weight occupies (codes + scales). */
size_t dj_weight_bytes(const dj_weight *w);

/* ---------------------------------------------------------------- recorder (gpu.ts:176-281) */

/* Starts recording a forward. graph_key == 0: ops are launched as they are recorded. graph_key != 0: the
 * forward is captured once into a HIP graph cached under that key; on later calls with the same key
 * *replay is set to 1, the host may skip the op calls (they are ignored) and dj_rec_finish relaunches
 * the graph. The key must change whenever a shape, a pointer or a scalar argument of any op changes.
 * Replaces: recorder() (gpu.ts:177-183). */
int dj_rec_begin(dj_ctx *ctx, uint64_t graph_key, dj_rec **out, int *replay);
/* Asynchronous host->device copy ordered before the recorder's ops (per-forward metadata: ids, meta,
 * leaves...). `host` is copied into pinned staging memory at once, so it may be reused on return.
 * Replaces: storage(view) (gpu.ts:148-152). Not allowed while capturing a graph: upload first. */
int dj_upload(dj_ctx *ctx, void *dev, const void *host, size_t bytes);
/* Asynchronous device->device copy on the context's stream (a kernel: it may be recorded into a graph).
 * Both pointers 16-byte aligned. Used to move inputs already resident in HBM into an engine's buffers. */
int dj_buf_copy(dj_ctx *ctx, void *dst_dev, const void *src_dev, size_t bytes);
/* Copies `bytes` of device memory into `host` once the forward has run (filled by dj_rec_finish).
 * Replaces: snapshot(buf, bytes, type) (gpu.ts:237-244). */
int dj_rec_snapshot(dj_rec *rec, const void *dev, size_t bytes, void *host);
/* Runs (or replays) the forward, waits for it, fills the snapshots, and frees the recorder.
 * Replaces: finish(tokens) (gpu.ts:245-279). */
int dj_rec_finish(dj_rec *rec);
/* Ends a forward whose recording failed (an op returned an error) without running what remains: nothing
 * more is launched, a partial capture becomes no graph, ops already launched are waited for, and the recorder's
 * temporaries are freed, so the next forward on the context starts clean. Replaces: finish()'s error path,
 * which destroys the forward's temporaries and throws (gpu.ts:255-260). */
int dj_rec_abort(dj_rec *rec);
/* Drops every cached graph (call after reallocating buffers a cached graph points to). */
int dj_graph_clear(dj_ctx *ctx);
/* Drops the graph cached under `key`, if any (call when memory one graph points to is freed, e.g. a shared
 * state's kept K/V). The cache also holds at most DJ_GRAPH_CAP graphs (default 64), evicting the least
 * recently used. No counterpart in the reference (WebGPU has no graphs); the hosts' shared-state free calls it. */
int dj_graph_drop(dj_ctx *ctx, uint64_t key);
/* Number of graphs in the cache (monitoring and tests). */
int dj_graph_count(dj_ctx *ctx, int *n);

/* ---------------------------------------------------------------- timing and profiling (gpu.ts:29-34, 185-197) */

/* HIP events on the context's stream around whatever is queued between begin and end; end waits. */
int dj_timer_begin(dj_ctx *ctx);
int dj_timer_end(dj_ctx *ctx, float *ms);
/* Per-kernel GPU time: when on, every op launch is bracketed by events and its time is added to a table
 * keyed by kernel name (the reference's globalThis.__d1Profile map). Ops in a captured graph are not
 * profiled. dj_profile_get copies up to `cap` entries and returns the count in *n. */
int dj_profile_enable(dj_ctx *ctx, int on);
typedef struct { char name[96]; double ms; int64_t launches; } dj_profile_entry;
int dj_profile_get(dj_ctx *ctx, dj_profile_entry *out, int cap, int *n);
int dj_profile_reset(dj_ctx *ctx);

/* ---------------------------------------------------------------- ops: embedding and norms */

/* X[t, :] = dequant(embed row ids[t]) in f16, X = f16(f16(code) - f16(zp)) * scale (RNE), t < T.
 * `embed` must be DJ_W_PLAIN, q8 or q4; ids past the vocabulary read its last row (as WebGPU's robust
 * buffer access keeps such reads in bounds). Replaces GATHER_Q8 / GATHER_Q4 (kernels.ts:6-21, 292-296). */
int dj_gather_q(dj_rec *rec, const uint32_t *ids_dev, int T, const dj_weight *embed, uint16_t *X_dev);

/* Per row t < T of H: if add, X += Y (stored f16); O = f16(f32(X) * rsqrt(mean(x^2) + eps) * w), where the
 * sum of squares uses the unrounded sum and the product the stored X.
 * Replaces ADD_RMSNORM (kernels.ts:23-46). */
int dj_add_rmsnorm(dj_rec *rec, int T, int H, int add, float eps, uint16_t *X_dev, const uint16_t *Y_dev,
                   const uint16_t *w_dev, uint16_t *O_dev);

/* Gemma sandwich norm per row: X = f16((X + rmsnorm(Y) * w1) * scale); if w2_dev, O = rmsnorm(f16 X) * w2.
 * Replaces SANDWICH (eg2-kernels.ts:15-48) for any H (the reference hard-codes 512). Y_dev may be NULL
 * (a zero branch: X is only renormalized, eg2-engine.ts:336). */
int dj_sandwich(dj_rec *rec, int T, int H, float eps, float scale, uint16_t *X_dev, const uint16_t *Y_dev,
                const uint16_t *w1_dev, const uint16_t *w2_dev, uint16_t *O_dev);

/* ---------------------------------------------------------------- ops: quantized matmul */

/* Y[M, N] = X[M, K] . W^T, f16 in and out, f32 accumulation on f16 MFMA, W dequantized in registers
 * exactly as the gather (bit-exact f16 weights). `w` must be DJ_W_MFMA. X rows are M (no padding needed).
 * Replaces recorder().matmul (gpu.ts:202-226) and MATMUL_Q8/Q4_SG32, MATMUL_DIRECT, matmulSplitK,
 * matmulPortable* (kernels.ts:298-385, 441-520, 545-768).
 * On a few rows (M <= 64, q8/q4, K long enough to split) the recorder may hold the product back by one
 * call: if the next op is dj_add_rmsnorm(add) of Y with T = M and H = N, the product runs split along K and
 * that norm sums its f32 partials (it also writes Y); any other op, snapshot, dj_rec_finish or stream-using
 * buffer call launches it first as an ordinary product. Y holds the product either way; a launch error
 * of a held product is reported by the call that launched it. DJ_GEMV_SPLIT=0 turns this off. */
int dj_matmul(dj_rec *rec, const uint16_t *X_dev, const dj_weight *w, uint16_t *Y_dev, int M);

enum { DJ_ACT_SILU = 0, DJ_ACT_GELU_TANH = 1, DJ_ACT_GELU_ERF = 2 };
/* Fused gated MLP input: for w = [w1; w3] (N = 2I, layout DJ_W_MFMA_GLU), Hout[M, I] =
 * f16(act(a) * b) with a = f16(X . w1^T), b = f16(X . w3^T) (rounded as the f16 matmul output).
 * act SILU: a / (1 + exp(-a)) (SILU_MUL / MATMUL_SWIGLU, kernels.ts:48-60, 591-599);
 * act GELU_TANH: 0.5 a (1 + tanh(0.7978845608 (a + 0.044715 a^3))), tanh argument clamped to +-15
 * (GELU_MUL, eg2-kernels.ts:9-13, 165-177);
 * act GELU_ERF: 0.5 a (1 + erf(a / sqrt 2)), erf by Abramowitz & Stegun 7.1.26 (|error| < 1.5e-7; Laya's
 * GELU_MUL, encoder-kernels.ts:25-41). Replaces recorder().swiglu (gpu.ts:229-234) and the separate GELU_MUL
 * dispatches. */
int dj_matmul_glu(dj_rec *rec, const uint16_t *X_dev, const dj_weight *w, uint16_t *H_dev, int M, int act);

/* ---------------------------------------------------------------- ops: q/k norm + rope, attention */

enum { DJ_ROPE_POW_NEG = 0,  /* ang = pos * pow(theta, -2d/rot)   (kernels.ts:106, d3-kernels.ts:172) */
       DJ_ROPE_INV_POW = 1   /* ang = pos * (1 / pow(theta, 2d/rot)) (eg2-kernels.ts:86) */ };
/* In place on fused rows Z[T, stride] holding [q heads | k heads | v heads] of D each:
 * per (token, q or k head) RMSNorm over D times qn / kn (skipped when the pointer is NULL: plain RoPE as
 * encoder-kernels.ts:5-23); if vnorm, v heads get a plain RMSNorm (eg2-kernels.ts:76-81); then half-split
 * (rotate-half) RoPE on the first `rot` dims (rot == D, or 64 with D = 256 as d3-kernels.ts:169) at
 * position pos[t * pos_stride]. f32 math, f16 store; the normed value is not rounded before RoPE.
 * Replaces QK_NORM_ROPE (kernels.ts:86-112), QK_NORM_ROPE_256 (d3-kernels.ts:151-178), ROPE
 * (encoder-kernels.ts:5-23), QKV_NORM_ROPE (eg2-kernels.ts:50-96), for any even D <= 512. */
int dj_qk_norm_rope(dj_rec *rec, int T, int heads, int kv, int D, int stride, uint16_t *Z_dev,
                    const uint16_t *qn_dev, const uint16_t *kn_dev, int vnorm, const int32_t *pos_dev,
                    int pos_stride, float eps, float theta, int rot, int rope_mode);

/* The (cos, sin) pairs dj_qk_norm_rope computes for each token, kept for a whole forward:
 * tab[t * rot/2 + i] = (cos a, sin a), a = f32(pos[t * pos_stride] * f_i), f_i as dj_qk_norm_rope (mode).
 * tab_dev holds T * rot/2 float pairs. The reference recomputes these angles in every layer's QK_NORM_ROPE
 * dispatch (kernels.ts:99-107); one table per forward feeds dj_matmul_qkv_rope in every layer. */
int dj_rope_table(dj_rec *rec, int T, const int32_t *pos_dev, int pos_stride, float theta, int rot, int rope_mode,
                  float *tab_dev);

/* recorder().matmul(X, w_qkv, Z, M) (gpu.ts:202-226) followed by QK_NORM_ROPE (kernels.ts:86-112) on Z: the
 * same results as dj_matmul then dj_qk_norm_rope(M, heads, kv, D, stride = w->N, Z, qn, kn, vnorm, pos,
 * pos_stride, eps, theta, rot, rope_mode) where that dj_matmul sums K in step order (its tiles with K wave
 * sets add two partial sums instead: the same product to within its f32 rounding). tab_dev: dj_rope_table of the same positions, theta, rot and mode
 * (M rows). For D = 128, M > 64 and at most two 128-row head tiles per CU the norm and rotation run in the
 * product's epilogue on tab_dev's angles (one head per tile, one kernel instead of two); otherwise as the two
 * kernels. */
int dj_matmul_qkv_rope(dj_rec *rec, const uint16_t *X_dev, const dj_weight *w, uint16_t *Z_dev, int M, int heads,
                       int kv, int D, const uint16_t *qn_dev, const uint16_t *kn_dev, int vnorm, const int32_t *pos_dev,
                       int pos_stride, float eps, float theta, int rot, int rope_mode, const float *tab_dev);

/* The residual add and RMSNorm between the decoder's products folded into them (d1-3b-engine.ts:98-104: the
 * o_proj and w2 products, each followed by ADD_RMSNORM, kernels.ts:23-46, whose output feeds the next product).
 *
 * dj_matmul_residual, the producer: with Y = f16(X . W^T) (rounded as dj_matmul's output),
 *   R[m, n] <- f16(R + Y)                       the residual stream, in place (ADD_RMSNORM's X)
 *   XW[m, n] = f16(R_new[m, n] * nw[n] / 4)     the norm weight applied, a quarter scale (no f16 overflow for
 *                                               norm weights up to 4)
 *   SS[m, b] = sum over the 32 columns of block b of (R + Y)^2, f32 on the unrounded sums (ADD_RMSNORM's
 *              sum of squares in parts), N / 32 floats per row.
 * Y itself is not stored. N % 32 == 0. */
int dj_matmul_residual(dj_rec *rec, const uint16_t *X_dev, const dj_weight *w, int M, uint16_t *R_dev,
                       const uint16_t *nw_dev, uint16_t *XW_dev, float *SS_dev);

/* dj_matmul_normed, the consumer: the product of the normalized rows, every output row m scaled by
 *   rs[m] = 4 / sqrt(sum_b SS[m, b] / H + eps)
 * before its f16 rounding: RMSNorm(R_new) . W^T with the norm weight applied before the product and 1 / rms
 * after (the same value as ADD_RMSNORM's O . W^T up to where the f16 roundings fall). XW and SS are
 * dj_matmul_residual's outputs with H its N (= this weight's K; H % 32 == 0, H <= 2048; above 1024, off
 * multiples of 128, or on 64 rows or fewer, the rows are normalized by a small kernel into the context workspace
 * first). act < 0: plain (DJ_W_MFMA weight); else the
 * gated epilogue of dj_matmul_glu (DJ_W_MFMA_GLU weight) on the scaled gate and up values. */
int dj_matmul_normed(dj_rec *rec, const uint16_t *XW_dev, const dj_weight *w, uint16_t *Y_dev, int M, int act,
                     const float *SS_dev, int H, float eps);

/* dj_matmul_qkv_rope on normalized rows (as dj_matmul_normed: XW, SS, H, norm_eps), the q/k norm and RoPE
 * applied to the scaled product. */
int dj_matmul_qkv_rope_normed(dj_rec *rec, const uint16_t *XW_dev, const dj_weight *w, uint16_t *Z_dev, int M,
                              int heads, int kv, int D, const uint16_t *qn_dev, const uint16_t *kn_dev, int vnorm,
                              const int32_t *pos_dev, int pos_stride, float eps, float theta, int rot, int rope_mode,
                              const float *tab_dev, const float *SS_dev, int H, float norm_eps);

/* Key/value source of dj_attention: `rows` rows of `stride` halves; K of kv head j at column k_col + j*D,
 * V at v_col + j*D. Key indices outside [0, rows) are clamped (never read out of bounds). */
typedef struct { const uint16_t *base; int rows; int stride; int k_col; int v_col; } dj_kv_src;

/* O[t, h*D + d] for t < T, h < heads: softmax(scale * q . k) . v over the keys of query t's two ranges
 * rng[t] = (a0, a1, b0, b1): key rows [a0, a1) of `kvA` and [b0, b1) of `kvB` (empty ranges allowed).
 * Q rows are Z[t * q_stride + h * D]. GQA: query head h reads kv head h / (heads / kv). f32 scores and
 * online softmax (m0 = -1e30), output f16(acc / l). This covers the causal forest of ATTENTION
 * (kernels.ts:114-147; mask of line 135 as ranges), the bidirectional/windowed ranges of eg2 attention
 * (eg2-kernels.ts:98-163) and the trunk+branch ranges of attention256 (d3-kernels.ts:180-240, without its
 * gate), and a kept prefix KV (kvA = the cache) for the shared-state mode. D in {64, 128, 256}; scale > 0
 * (the reference's 1/sqrt(D), or 1 for eg2), else DJ_EINVAL. */
int dj_attention(dj_rec *rec, int T, int heads, int kv, int D, const uint16_t *Q_dev, int q_stride,
                 dj_kv_src kvA, dj_kv_src kvB, const int32_t *rng_dev, float scale, uint16_t *O_dev);

/* QK_NORM_ROPE (kernels.ts:86-112) on the query heads of Q and the key heads of source B, folded into
 * dj_attention (kernels.ts:114-147), i.e. the pair of dispatches at d1-3b-engine.ts:95-96: the same results as dj_qk_norm_rope(T, heads, kv, 128, stride, Z, qn, kn,
 * 0, pos, ...) on the fused rows, then dj_attention, except that Z keeps its raw q and k values. The angles come
 * from tab_dev (dj_rope_table of the same T rows and positions, rot 128); source B must be the T query rows
 * themselves (kvB.rows == T, its row t rotated with tab row t) and source A already normalized and rotated (a
 * kept state). D = rot = 128 (else DJ_EINVAL). The short-question form of the forward: the qkv product then
 * this, one launch fewer per layer than dj_qk_norm_rope + dj_attention. */
int dj_attention_qk_rope(dj_rec *rec, int T, int heads, int kv, int D, const uint16_t *Q_dev, int q_stride,
                         dj_kv_src kvA, dj_kv_src kvB, const int32_t *rng_dev, float scale, const uint16_t *qn_dev,
                         const uint16_t *kn_dev, float eps, const float *tab_dev, int rot, uint16_t *O_dev);

/* dj_attention that allocates nothing, for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid it). No counterpart in the reference. Same arguments and
 * results as dj_attention; its split-KV partials (a short question against a long kept state) live in the
 * library's static device scratch of 8 MiB per GPU instead of the context's workspace. A call whose split plan
 * needs more than that (splits * T * heads * (D + 2) f32) is refused with DJ_EINVAL. Every call on a GPU shares
 * that GPU's scratch: calls that overlap on one GPU race. */
int dj_attention_noalloc(dj_rec *rec, int T, int heads, int kv, int D, const uint16_t *Q_dev, int q_stride,
                         dj_kv_src kvA, dj_kv_src kvB, const int32_t *rng_dev, float scale, uint16_t *O_dev);

/* Copies K and V of rows [0, T) of the fused rows Z into cache rows [row0, row0 + T) of layout
 * [rows, 2 * kv * D] (K heads then V heads): the kept KV of a prefilled shared state. */
int dj_kv_store(dj_rec *rec, int T, int kv, int D, const uint16_t *Z_dev, int stride, int k_col,
                uint16_t *cache_dev, int row0);

/* ---------------------------------------------------------------- ops: LFM2 short conv */

/* Y[t, c] = f16(C[t, c] * sum_j w[c, j] * B[tap_j, c] * U[tap_j, c]) for the fused in_proj rows
 * Z[T, 3H] = [B | C | U] and conv taps w f16 [H, 3] (the depthwise conv weight), products in f32; taps i32
 * [T, 4] names the tokens taps 0..2 read (-1 or >= T: zero; the 4th is unused): (t-2, t-1, t) for d1-3B's
 * causal forest, a branch continuing its trunk, or (t-1, t, t+1) within a sequence for d1-omni. H % 8 == 0.
 * Replaces SHORT_CONV (kernels.ts:62-84). */
int dj_short_conv(dj_rec *rec, int T, int H, const uint16_t *Z_dev, const uint16_t *w_dev, const int32_t *taps_dev,
                  uint16_t *Y_dev);

/* ---------------------------------------------------------------- ops: d3-lite's mixers (d3-kernels.ts) */

/* The Gated DeltaNet mixer after the in-projection, for every (sequence, head) (gdnLayer, d3-kernels.ts:9-149):
 * Z [T, stride] f16 rows q | k | v | z (LH x 128 each) | b | a (LH each); conv_w f16 [3 LH 128, 4] (causal taps,
 * tap 3 the token itself); A_log, dt_bias f16 [LH]; gnorm f16 [128]. spans (device, u32 [nspans, 4]): (a start,
 * a length | write_a << 31, b start, b length): a sequence is span a then span b (a shared trunk rescanned by
 * each question, then the question; or the whole sequence and an empty b); span a's outputs are written only
 * when write_a is set. Y [T, LH 128] f16 = gated RMSNorm (eps) of the delta rule's output. Key and value heads
 * are 128 wide and equal in number; the conv has 4 taps. Replaces dispatch(gdnLayer(...)) (d3-engine.ts:116). */
int dj_gdn(dj_rec *rec, int T, int nspans, const uint32_t *spans_dev, int LH, int stride, const uint16_t *Z_dev,
           const uint16_t *conv_w_dev, const uint16_t *A_log_dev, const uint16_t *dt_bias_dev,
           const uint16_t *gnorm_dev, float eps, uint16_t *Y_dev);
/* dj_attention with d3's output gate: O = f16(attention / (1 + exp(-G[t, h D + d]))), G rows of g_stride halves
 * (the gate heads of the fused q | k | v | gate rows). Replaces attention256 (d3-kernels.ts:180-240). */
int dj_attention_gated(dj_rec *rec, int T, int heads, int kv, int D, const uint16_t *Q_dev, int q_stride, dj_kv_src A,
                       dj_kv_src B, const int32_t *rng_dev, float scale, const uint16_t *G_dev, int g_stride,
                       uint16_t *O_dev);

/* ---------------------------------------------------------------- ops: EmbeddingGemma 2's per-layer embeddings */

/* O[t, :] = f16(gelu_tanh(G[t, :]) * E[t, :] / sqrt(mean(E[t, :]^2) + eps) * w), G, E, O f16 [T, P], w f16 [P],
 * P % 8 == 0. Replaces PLE_MIX (eg2-kernels.ts:179-200). */
int dj_ple_mix(dj_rec *rec, int T, int P, const uint16_t *G_dev, const uint16_t *E_dev, const uint16_t *w_dev, float eps,
               uint16_t *O_dev);
/* out[s, :] = mean(X[a_s:b_s, :]) . W^T in f32, W f16 [N, H] (the embedding projection), seqs (a, b) per
 * sequence; H % 4 == 0. The mean is staged in the context workspace. Replaces POOL_PROJECT (eg2-kernels.ts:202-228). */
int dj_pool_project(dj_rec *rec, int T, int S, int H, int N, const uint16_t *X_dev, const uint32_t *seqs_dev,
                    const uint16_t *W_dev, float *out_dev);

/* ---------------------------------------------------------------- ops: d1-omni's decision head (kernels.ts:186-283) */

/* Xo[t, :] = f16(f32(Xi[t, :]) + f32(E[idx[t], :])) for E f16 [rows, H] (the question-type embedding); idx past
 * the table reads its last row. H % 8 == 0. Replaces ADD_ROWS (kernels.ts:188-201). */
int dj_add_rows(dj_rec *rec, int T, int H, const uint16_t *Xi_dev, const uint32_t *idx_dev, const uint16_t *E_dev,
                int rows, uint16_t *Xo_dev);
enum { DJ_BIAS_NONE = 0, DJ_BIAS_RELU = 1, DJ_BIAS_GELU_ERF = 2 };
/* Y[t, n] = f16(act(f32(Y[t, n]) + f32(b[n]))) in place, act none / ReLU / GELU with the Abramowitz & Stegun
 * 7.1.26 erf. N % 8 == 0. Replaces BIAS_ACT (kernels.ts:203-222). */
int dj_bias_act(dj_rec *rec, int T, int N, uint16_t *Y_dev, const uint16_t *b_dev, int act);
/* Per row: if add, X += Y (stored f16); O = f16((f32(X) - mean) / sqrt(max(E[x^2] - mean^2, 0) + eps) * w + b)
 * with the mean and E[x^2] of the unrounded sum. H % 8 == 0. Replaces ADD_LAYERNORM (kernels.ts:224-255). */
int dj_add_layernorm(dj_rec *rec, int T, int H, int add, float eps, uint16_t *X_dev, const uint16_t *Y_dev,
                     const uint16_t *w_dev, const uint16_t *b_dev, uint16_t *O_dev);
/* G[m, :] = X[rows[m], :] for m < M (rows clamped to [0, T)). Replaces GATHER_ROWS (kernels.ts:257-267). */
int dj_gather_rows(dj_rec *rec, int M, int H, int T, const uint16_t *X_dev, const uint32_t *rows_dev, uint16_t *G_dev);
/* out[m] = Y[m, :] . w + b[0] in f32 (the scorer's last Linear(H, 1)). Replaces SCORE (kernels.ts:269-283). */
int dj_score(dj_rec *rec, int M, int H, const uint16_t *Y_dev, const uint16_t *w_dev, const uint16_t *b_dev, float *out_dev);

/* ---------------------------------------------------------------- ops: readouts and pooling */

/* out[l * nIds + j] = rmsnorm_f32(X[leaves[l]]) * w  .  dequant_f32(embed row ids[l * nIds + j]) in f32:
 * the final norm is recomputed in f32 (not rounded) and the embedding dequantized in f32
 * ((f32(code) - zp) * f32(scale)). embed q8 or q4, DJ_W_PLAIN. Replaces LEAF_LOGITS (kernels.ts:149-185),
 * which is q4-only with H <= 2048 in the reference. Leaf rows are clamped to [0, T), ids to the vocabulary. */
int dj_leaf_logits(dj_rec *rec, int T, int L, int H, int nIds, float eps, const uint16_t *X_dev,
                   const uint32_t *leaves_dev, const uint16_t *w_dev, const uint32_t *ids_dev,
                   const dj_weight *embed, float *out_dev);

/* out[k] = X[pairs[2k]] . R[pairs[2k+1]] in f32 (R f32 [codes, H]). Replaces READOUT (d3-kernels.ts:242-260). */
int dj_readout(dj_rec *rec, int T, int P, int H, const uint16_t *X_dev, const float *R_dev, int codes,
               const uint32_t *pairs_dev, float *out_dev);

/* out[s, :] = mean of X rows [seqs[2s], seqs[2s+1]) in f32. The pooling half of POOL_PROJECT
 * (eg2-kernels.ts:202-228), for any H. */
int dj_mean_pool(dj_rec *rec, int T, int S, int H, const uint16_t *X_dev, const uint32_t *seqs_dev, float *out_dev);

/* out[M, N] = in[M, K] . dequant_f32(W)^T in f32 (f32 activations, weights as LEAF_LOGITS dequantizes them),
 * for the small dense head after pooling (the projection half of POOL_PROJECT, generalised). W DJ_W_PLAIN. */
int dj_dense_f32(dj_rec *rec, int M, const float *in_dev, const dj_weight *w, float *out_dev);

#ifdef __cplusplus
}
#endif
#endif /* DJ_H */
