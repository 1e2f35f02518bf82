/*
 * laya_hip.h -- C ABI of libhipbackend.so, the MI355X (gfx950) device layer
 * behind laya-js' `Backend<T>` contract
 * (packages/tensor-backend/src/index.ts:139-317).
 *
 * The host side (a TypeScript backend-hip over koffi / bun:ffi, or the
 * Python mirror in laya-js_amd/laya_hip) owns tensor metadata -- shape,
 * dtype, strides, views, scopes -- and calls these functions with plain
 * device addresses and sizes.  This is the same split as the reference's
 * mlx-c binding (packages/backend-mlx/src/ffi.ts:31-114): no C++ or torch
 * types cross the boundary.
 *
 * Conventions
 *  - Handles and device addresses are uintptr_t.
 *  - Every function returns 0 on success and -1 on failure; it never aborts
 *    the process.  hb_last_error() then returns the message (thread-local),
 *    which the host raises as an Error naming the op (the reference's
 *    failure rule: packages/backend-mlx/src/ffi.ts:15-16,190-201).
 *  - A context owns one HIP stream.  Ops enqueue on it and return at once;
 *    hb_download / hb_sync / hb_event_elapsed wait.  A context is used from
 *    one host thread at a time (the contract is single-threaded,
 *    tensor-backend/src/index.ts:5-10).
 *  - Element strides (not bytes) describe strided operands; a stride of 0
 *    broadcasts.  dtype codes are HB_F32 ... below.
 */
#ifndef LAYA_HIP_H
#define LAYA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HB_ABI_VERSION 1

/* dtype codes: the contract's DType names (tensor-backend/src/index.ts:39). */
enum {
  HB_F32 = 0,
  HB_F16 = 1,
  HB_BF16 = 2,
  HB_I32 = 3,
  HB_BOOL = 4, /* one byte, 0/1 */
  HB_U8 = 5,
  HB_I8 = 6,
  HB_U16 = 7,
  HB_I16 = 8,
  HB_U32 = 9
};

/* hb_linear / hb_qlinear epilogue flags */
#define HB_EPI_BIAS 1u  /* y += bias[n] (f32 add before the one rounding) */
#define HB_EPI_RESID 2u /* y = round(round(x.w^T) + resid): linear then add, as two contract ops */
#define HB_EPI_GEGLU 4u /* w has 2N rows; y[:, j] = gelu(round(h[:, j])) * round(h[:, N + j]) */
#define HB_X_PANEL 8u   /* x is in panel order (below); ldx is ignored */
#define HB_Y_PANEL 16u  /* y is written in panel order; ldy is ignored */

/* Panel order of a 16-bit [M, K] matrix (K % 16 == 0), an internal layout
 * for activations that feed a large-M linear layer: the matrix is cut into
 * 32-row x 16-column blocks of 1 KB, block (i, j) at element offset
 * (i * (K/16) + j) * 512; inside a block, 16-byte chunk c = 32*h + r holds
 * row 32*i + r, columns 16*j + 8*h ... 16*j + 8*h + 7.  This is the operand
 * order of v_mfma_f32_32x32x16 (lane l reads chunk l), so the GEMM loads one
 * whole block per instruction instead of 32 bytes of 32 rows.  Storage holds
 * ceil(M/32)*32 rows; rows M... of the last block are padding. */

/* hb_unary ops (tensor-backend/src/index.ts:177-198, 265-300) */
enum {
  HB_UN_COPY = 0, /* strided copy / cast into a contiguous output */
  HB_UN_SCALE = 1,
  HB_UN_EXP = 2,
  HB_UN_LOG = 3,
  HB_UN_RELU = 4,
  HB_UN_GELU = 5,
  HB_UN_NEG = 6,
  HB_UN_ABS = 7,
  HB_UN_SQRT = 8,
  HB_UN_RSQRT = 9,
  HB_UN_TANH = 10,
  HB_UN_SIGMOID = 11,
  HB_UN_ERF = 12,
  HB_UN_NOT = 13
};

/* hb_binary ops (tensor-backend/src/index.ts:180-191, 269-291) */
enum {
  HB_BIN_ADD = 0,
  HB_BIN_SUB = 1,
  HB_BIN_MUL = 2,
  HB_BIN_DIV = 3,
  HB_BIN_MAX = 4,
  HB_BIN_MIN = 5,
  HB_BIN_POW = 6,
  HB_BIN_EQ = 7,
  HB_BIN_NE = 8,
  HB_BIN_LT = 9,
  HB_BIN_LE = 10,
  HB_BIN_GT = 11,
  HB_BIN_GE = 12,
  HB_BIN_AND = 13,
  HB_BIN_OR = 14
};

/* ---------------------------------------------------------------- runtime */

/* Message of the last failed call on this thread ("" if none). */
const char* hb_last_error(void);
int hb_abi_version(void);

/* Opens device `device` and creates a context with one stream.
 * Replaces createMlxBackend's device/stream setup (backend-mlx/src/index.ts:920).
 * It makes `device` current on the calling thread.  A context's later calls
 * need that device current: calls that would create device memory or events
 * fail with an error while another device is current. */
int hb_init(int device, uintptr_t* ctx);
/* Frees every pooled block and the stream.  Backend.destroy (index.ts:165-166). */
int hb_destroy(uintptr_t ctx);
/* JSON: {"name","arch","cus","hbm_bytes","lds_per_cu","clock_khz",...}. */
int hb_device_info(uintptr_t ctx, char* buf, size_t cap);

/* Stream-ordered pooled device memory (blocks are 256-byte aligned).  A
 * block freed with hb_free is reused only by work enqueued later on the same
 * stream, so it is safe to free right after enqueueing its last reader.
 * Backs fromHost / op outputs / dispose (index.ts:153-157). */
int hb_alloc(uintptr_t ctx, size_t bytes, uintptr_t* ptr);
int hb_free(uintptr_t ctx, uintptr_t ptr);
/* live bytes, cached (free) bytes, live block count */
int hb_pool_stats(uintptr_t ctx, uint64_t* live_bytes, uint64_t* cached_bytes, uint64_t* live_blocks);
/* Returns cached blocks to the driver (after a stream sync). */
int hb_pool_trim(uintptr_t ctx);

/* Copies `bytes` from host memory into device memory.  The host buffer is
 * copied into pinned staging before the call returns, so the caller may
 * reuse it at once (fromHost's copy-at-call rule, index.ts:146-153). */
int hb_upload(uintptr_t ctx, uintptr_t dst, const void* src, size_t bytes);
/* Waits for the stream, then copies device -> host (Backend.read, index.ts:154-155). */
int hb_download(uintptr_t ctx, void* dst, uintptr_t src, size_t bytes);
/* Device-to-device copy on the stream. */
int hb_copy(uintptr_t ctx, uintptr_t dst, uintptr_t src, size_t bytes);
/* Fills `bytes` with the byte `value` using a kernel (graph-capture safe). */
int hb_fill(uintptr_t ctx, uintptr_t dst, int value, size_t bytes);
/* Waits until every op enqueued on the context has finished (Backend.flush). */
int hb_sync(uintptr_t ctx);

/* HIP events on the context's stream, for timing (the reference's
 * Runtime.startProfiling/stopProfiling timestamps, backend-webgpu/src/runtime.ts:420-464). */
int hb_event_create(uintptr_t ctx, uintptr_t* ev);
int hb_event_record(uintptr_t ctx, uintptr_t ev);
/* Waits for `end`, then writes the milliseconds between the two records. */
int hb_event_elapsed(uintptr_t start, uintptr_t end, float* ms);
int hb_event_destroy(uintptr_t ev);

/* Stream capture.  No counterpart in the reference's Backend: for callers
 * that run the same op sequence again and again on small batches, where the
 * host's per-op launches, not the GPU, bound the time.
 * hb_capture_begin starts recording the context's stream (relaxed mode);
 * the ops enqueued until hb_capture_end are recorded, not run, and
 * hb_capture_end instantiates them as an executable graph.  hb_graph_launch
 * replays it on the stream: the same kernels on the same device addresses,
 * so the caller keeps the recorded inputs and outputs alive and rewrites
 * inputs in place between replays.  Blocks freed while recording stay out
 * of the pool until hb_graph_destroy.  Between begin and end: no
 * hb_upload / hb_download / hb_sync, and no op whose one-time set-up uploads
 * (run the sequence once before recording it). */
int hb_capture_begin(uintptr_t ctx);
int hb_capture_end(uintptr_t ctx, uintptr_t* exec);
int hb_graph_launch(uintptr_t ctx, uintptr_t exec);
int hb_graph_destroy(uintptr_t ctx, uintptr_t exec);

/* ---------------------------------------------------------------- hot path */

/* y[M, N] = x[M, K] . w[N, K]^T with f32 accumulation and the epilogue in
 * `flags`.  Backend.linear (tensor-backend/src/index.ts:211-215) reached
 * through compose.linearAny (compose.ts:431-433); HB_EPI_RESID fuses the
 * following Backend.add (modernbert/src/index.ts:353,355) and HB_EPI_GEGLU
 * the following compose.geglu (compose.ts:86-93, modernbert index.ts:354-355).
 *  dt     HB_F16 / HB_BF16 (MFMA path) or HB_F32 (f32 path); x, w, y,
 *         resid and bias share it.
 *  ldx    row stride of x in elements (>= K); ldy of y; ldr of resid.
 *  GEGLU: w has 2N rows (value rows 0..N-1, gate rows N..2N-1), y has N
 *         columns; bias (if any) has 2N entries. */
int hb_linear(uintptr_t ctx, int dt, uintptr_t x, int64_t ldx, uintptr_t w, uintptr_t bias, uintptr_t resid,
              int64_t ldr, uintptr_t y, int64_t ldy, int64_t M, int64_t N, int64_t K, unsigned flags);
/*  HB_X_PANEL / HB_Y_PANEL (hb_linear and hb_qlinear): x read from / y
 *  written in panel order.  Taken by two kernels: dt f16 or bf16,
 *  K % 64 == 0, 16-byte aligned operands, and either M >= 4096 (the large-M
 *  kernel), or, for hb_linear only, a call that takes the small-M slab
 *  kernel: 64 * K * (2 with GeGLU) <= 160 KiB and
 *  ceil(N / 32) * ceil(M / 128) <= the device's CUs (hb_device_info "cus").
 *  A panel-order y also needs N % 16 == 0 and no residual.  Other calls
 *  fail.  The arithmetic is the same as with row-major operands, bit for
 *  bit. */

/* The attention block's q / k / v projection fused with its layout glue
 * and RoPE: y = x . w^T for the stacked projection w [3*H*64, K] (no bias,
 * as ModernBERT's attention_bias = false; `bias` must be 0),
 * written head-major as y[3][B][H][L][64] (B = M / L, rows of x ordered
 * b * L + t), with the split-half rotation of base `rope_base` applied to the
 * q and k parts (none when rope_base <= 0), each value rounded to dt after
 * the product and again after the rotation -- bit for bit what
 * Backend.linear (tensor-backend/src/index.ts:211-215), reshape / transpose /
 * split (index.ts:169-176) and Backend.rope (index.ts:225-229) store when
 * called as modernbert/src/index.ts:348-351 does.
 *  dt     HB_F16 / HB_BF16 (x, w, y).
 *  Needs M >= 4096, K % 64 == 0, M % L == 0, 16-byte aligned operands;
 *  flags: HB_X_PANEL (x in panel order) only. */
int hb_linear_qkv(uintptr_t ctx, int dt, uintptr_t x, int64_t ldx, uintptr_t w, uintptr_t bias, uintptr_t y,
                  int64_t M, int64_t K, int64_t L, int64_t H, double rope_base, unsigned flags);

/* Quantized linear: y = x . dequant(W)^T (+ epilogue), W [N, K] in the
 * laya-js quantized layout v1 (HostQuantized, tensor-backend/src/index.ts:98-115;
 * docs/QUANTIZATION.md "Format"): `qw` row-major packed bytes, K*bits/8 per
 * row (4-bit: even column in the low nibble); `scales` and (affine)
 * `zeros` are f16 [N, ceil(K/group)].  Weights dequantize to
 * fl16(q*s + z) (fl16(q*s) when symmetric), exactly what host
 * dequantization uploads, and feed the f16 MFMA with f32 accumulation
 * (M >= 4096, and M >= 1024 for calls that neither the small-M slab
 * kernel nor 128 x 64 tiles take: once per call into a 16-bit copy taken
 * from the context's pool for the duration of the call; otherwise inside
 * the GEMM kernels' weight loaders).
 * Backend.quantizedLinear (index.ts:257-261) via compose.quantizedLinear
 * (compose.ts:407-414).
 *  dt     dtype of x / y / resid / bias: HB_F16, HB_BF16 or HB_F32.
 *  bits   8 or 4;  mode 0 = symmetric (signed q), 1 = affine (unsigned q). */
int hb_qlinear(uintptr_t ctx, int dt, uintptr_t x, int64_t ldx, uintptr_t qw, uintptr_t scales, uintptr_t zeros,
               uintptr_t bias, uintptr_t resid, int64_t ldr, uintptr_t y, int64_t ldy, int64_t M, int64_t N, int64_t K,
               int bits, int group, int mode, unsigned flags);

/* Row-gather of dequant(W) by ids: out [n, K] in dt_out.  Backend.quantizedEmbedding
 * (index.ts:262-263), compose.ts:417-428. */
int hb_qgather(uintptr_t ctx, uintptr_t qw, uintptr_t scales, uintptr_t zeros, int64_t V, int64_t K, int bits,
               int group, int mode, uintptr_t ids, int64_t n, int dt_out, uintptr_t out);

/* LayerNorm over the last axis of x [rows, D] (row stride ldx), f32
 * two-pass statistics; w / b may be 0.  Backend.layerNorm (index.ts:216-217). */
int hb_layernorm(uintptr_t ctx, int dt_x, uintptr_t x, int64_t ldx, int dt_w, uintptr_t w, uintptr_t b, int dt_y,
                 uintptr_t y, int64_t rows, int64_t D, float eps);

/* hb_layernorm with y (of x's dtype) written in panel order, for a
 * LayerNorm whose consumer is a large-M linear layer (the encoder's
 * attn_norm -> Wqkv and mlp_norm -> Wi, modernbert/src/index.ts:347-354).
 * Same arithmetic as hb_layernorm's 16-bit path, bit for bit; needs dt_x
 * f16 or bf16, D % 256 == 0, D <= 2048, ldx % 8 == 0, x and y 16-byte aligned and
 * the parameters aligned for 4-wide loads (8 bytes; 16 for f32).  Padding
 * rows of the last block are written as zeros. */
int hb_layernorm_panel(uintptr_t ctx, int dt_x, uintptr_t x, int64_t ldx, int dt_w, uintptr_t w, uintptr_t b,
                       uintptr_t y, int64_t rows, int64_t D, float eps);

/* Conversions between row-major (row stride ld) and panel order for a
 * 16-bit [M, K] matrix, K % 16 == 0: the host materialises a row-major
 * tensor from a panel-order one when an op other than a linear layer reads
 * it.  Buffers must be 16-byte aligned, ld % 8 == 0; hb_panel_pack writes
 * the padding rows as zeros. */
int hb_panel_pack(uintptr_t ctx, uintptr_t src, int64_t ld, uintptr_t dst, int64_t M, int64_t K);
int hb_panel_unpack(uintptr_t ctx, uintptr_t src, uintptr_t dst, int64_t ld, int64_t M, int64_t K);

/* Split-half RoPE on x [B, H, L, D] addressed by element strides xs[4];
 * y is contiguous [B, H, L, D].  Angles follow the f32 rule of the CPU
 * backend (backend-webgpu/src/backend.ts:1185-1195).  Backend.rope
 * (index.ts:225-229). */
int hb_rope(uintptr_t ctx, int dt_x, uintptr_t x, const int64_t* xs, int dt_y, uintptr_t y, int64_t B, int64_t H,
            int64_t L, int64_t D, double base);

/* Scaled dot-product attention, softmax in f32 (Backend.sdpa, index.ts:230-237).
 * q [B,H,Lq,D], k/v [B,H,Lk,D] and o [B,H,Lq,D] by element strides (4
 * each, last must be 1 for the MFMA path); mask is bool (1 byte) addressed
 * by ms[4] over [B,H,Lq,Lk] (0 = broadcast), or 0 for none.
 * mask_info: 0, or the summary hb_sdpa_mask_info wrote for this very mask
 * (and B, Lq, Lk), so a mask reused by many layers is summarised once.
 * rope_q / rope_k: when > 0, q (k) is first rotated by RoPE with that base
 * and rounded to dt, exactly as a preceding Backend.rope would
 * (modernbert/src/index.ts:351). */
int hb_sdpa(uintptr_t ctx, int dt, uintptr_t q, const int64_t* qs, uintptr_t k, const int64_t* ks, uintptr_t v,
            const int64_t* vs, uintptr_t mask, const int64_t* ms, uintptr_t mask_info, uintptr_t o, const int64_t* os,
            int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, float scale, double rope_q, double rope_k);

/* hb_sdpa with o written in panel order (HB_X_PANEL above) as the [B*Lq,
 * H*D] matrix whose row b*Lq + l holds the heads side by side: the layout
 * modernbert's transpose + reshape of the attention output
 * (modernbert/src/index.ts:352) feeds to attn Wo, for a large-M Wo that reads
 * it with HB_X_PANEL.  Same arithmetic as hb_sdpa; needs its MFMA path
 * (f16/bf16, D = 64, aligned operands, a mask that does not vary over heads)
 * and a 16-byte aligned o of ceil(B*Lq/32)*32 rows. */
int hb_sdpa_panel(uintptr_t ctx, int dt, uintptr_t q, const int64_t* qs, uintptr_t k, const int64_t* ks, uintptr_t v,
                  const int64_t* vs, uintptr_t mask, const int64_t* ms, uintptr_t mask_info, uintptr_t o, int64_t B,
                  int64_t H, int64_t Lq, int64_t Lk, int64_t D, float scale, double rope_q, double rope_k);
/* hb_sdpa without RoPE (rope_q = rope_k = 0) that allocates nothing: no
 * hipMalloc, no pool block.  No counterpart in the reference; it is for
 * callers that cannot allocate (code recorded into a HIP graph, tight
 * serving loops, harnesses that forbid allocation).  With a mask on the MFMA
 * path, the mask summary is built into a 2 MiB device array the library
 * holds per GPU until the process ends, so B * ceil(Lq/128) * ceil(Lk/64)
 * * 8 must not exceed 2097152 bytes (B = 32 at Lq = Lk = 8192); larger
 * shapes are refused with an error before anything is launched.  Every
 * call on one GPU shares that array: calls that overlap on one GPU (from
 * contexts with different streams) race; calls on one context's stream are
 * ordered.  Results are hb_sdpa's, bit for bit. */
int hb_sdpa_noalloc(uintptr_t ctx, int dt, uintptr_t q, const int64_t* qs, uintptr_t k, const int64_t* ks,
                    uintptr_t v, const int64_t* vs, uintptr_t mask, const int64_t* ms, uintptr_t o, const int64_t* os,
                    int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, float scale);
/* Size of a mask summary for (B, Lq, Lk). */
int hb_sdpa_mask_info_bytes(int64_t B, int64_t Lq, int64_t Lk, size_t* bytes);
/* Summarises a bool attention mask (strides ms[4] over [B,H,Lq,Lk], head
 * stride ignored) into `info`: for every (batch, 128-query, 64-key) tile
 * whether no key, every key or some keys are visible.  Enqueued on the
 * context's stream; `info` must stay alive while hb_sdpa calls use it. */
int hb_sdpa_mask_info(uintptr_t ctx, uintptr_t mask, const int64_t* ms, int64_t B, int64_t Lq, int64_t Lk,
                      uintptr_t info);

/* gelu(value) * gate over x [rows, 2F] (row stride ldx) -> y [rows, F].
 * Backend.geglu (index.ts:240-241), compose.ts:86-93. */
int hb_geglu(uintptr_t ctx, int dt_x, uintptr_t x, int64_t ldx, int dt_y, uintptr_t y, int64_t rows, int64_t F);

/* ---------------------------------------------------------------- generic ops */

/* y = op(x) over shape[rank], x addressed by strides xs and y by ys
 * (ys = NULL: y contiguous).  HB_UN_COPY is the strided copy / cast behind
 * reshape-of-a-view, transpose, slice, concat and cast (index.ts:169-177).
 * alpha is the scalar of HB_UN_SCALE. */
int hb_unary(uintptr_t ctx, int op, int dt_x, uintptr_t x, const int64_t* xs, int dt_y, uintptr_t y,
             const int64_t* ys, const int64_t* shape, int rank, double alpha);
/* y = a op b with numpy broadcasting expressed as strides (0 = broadcast);
 * arithmetic in f32 for float dtypes, i32 for integers.  Comparisons and
 * logical ops write bool.  Backend.add/sub/mul/div/maximum (index.ts:180-189). */
int hb_binary(uintptr_t ctx, int op, int dt_a, uintptr_t a, const int64_t* as, int dt_b, uintptr_t b,
              const int64_t* bs, int dt_y, uintptr_t y, const int64_t* shape, int rank);
/* y = cond ? a : b (Backend.where, index.ts:190-191). */
int hb_where(uintptr_t ctx, uintptr_t cond, const int64_t* cs, int dt_a, uintptr_t a, const int64_t* as, int dt_b,
             uintptr_t b, const int64_t* bs, int dt_y, uintptr_t y, const int64_t* shape, int rank);
/* Row gather: out[r, :] = table[ids[r], :] (Backend.embedding, index.ts:218-219);
 * with batch_rows > 0, row r reads table + (r / batch_rows) * V * D
 * (Backend.gatherRows, index.ts:220-224).  ids are clamped to [0, V). */
int hb_gather(uintptr_t ctx, int dt, uintptr_t table, int64_t V, int64_t D, uintptr_t ids, int64_t n,
              int64_t batch_rows, int dt_out, uintptr_t out);
/* hb_reduce / hb_scan ops (tensor-backend/src/index.ts:200-206, 301-316) */
enum {
  HB_RED_SUM = 0,
  HB_RED_MAX = 1,
  HB_RED_MIN = 2,
  HB_RED_MEAN = 3,
  HB_RED_ARGMAX = 4,
  HB_RED_ARGMIN = 5
};
enum { HB_SCAN_SOFTMAX = 0, HB_SCAN_CUMSUM = 1, HB_SCAN_SORT = 2 };

/* Reduces axis n of x viewed as [outer, n, inner] (contiguous) into y
 * [outer, inner]: sum / max / min / mean accumulate in f32 (i32 for integer
 * sum/max/min), argmax / argmin write the i32 index of the first extremum.
 * Backend.sum / max (index.ts:201-202), mean / min / argmax / argmin
 * (index.ts:301-308). */
int hb_reduce(uintptr_t ctx, int op, int dt_x, uintptr_t x, int64_t outer, int64_t n, int64_t inner, int dt_y,
              uintptr_t y);
/* Per-slice ops along axis n of [outer, n, inner] (contiguous) into y of the
 * same shape: softmax in f32 (index.ts:203-204), inclusive cumsum wrapping in
 * the output dtype (index.ts:309-316), ascending sort (index.ts:205-206). */
int hb_scan(uintptr_t ctx, int op, int dt_x, uintptr_t x, int64_t outer, int64_t n, int64_t inner, int dt_y,
            uintptr_t y);

/* Masked mean over axis 1: x [B, L, D], mask bool [B, L] -> f32 [B, D]
 * (Backend.meanPool, index.ts:242-243; compose.ts:96-105). */
int hb_meanpool(uintptr_t ctx, int dt_x, uintptr_t x, uintptr_t mask, int64_t B, int64_t L, int64_t D, uintptr_t out);

#ifdef __cplusplus
}
#endif

#endif /* LAYA_HIP_H */
