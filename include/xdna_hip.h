/* xdna_hip.h -- C ABI of the MI355X (gfx950) int8 hot path of torch_xdna.
 *
 * The reference (AyaSakura-comp/torch-xdna) reaches its device through Python launchers:
 * `kernels.mm_i8` (torch_xdna/kernels.py:172-192) for the int8 GEMM and Triton-XDNA's
 * `tl.extra.npu.conv3x3` op (called at torch_xdna/conv.py:78-84, :94-96) for the conv, with the
 * quantize / dequantize around them done as torch CPU ops (torch_xdna/runtime.py:145-148,
 * :350-353, :366-374; torch_xdna/conv.py:45-51). This library replaces all of them with HIP
 * kernels behind plain C entry points: every pointer is device memory the caller owns (torch's
 * caching allocator in torch_xdna), every size is an element count, every function enqueues on
 * the given hipStream_t (passed as void*) and returns an int status without synchronizing.
 *
 * Status: 0 = success; > 0 = a hipError_t from the launch; < 0 = an XDNA_E* code below. The
 * message of the last failure on the calling thread is xdna_last_error().
 *
 * Layout conventions: matrices are row-major with an explicit leading dimension (elements
 * between rows). int8 GEMM operands are "K-contiguous": A is [M, K], the weight is [N, K]
 * (one row per output channel). Operand rows must start on 16-byte boundaries and K must be a
 * multiple of 16 (the quantize entry points zero-pad K for this). Conv activations are NHWC with
 * the channel count padded to a multiple of 16 (`c_pad`), conv weights are [Co][9][ci_pad] with
 * taps in (ky, kx) order.
 */
#ifndef XDNA_HIP_H
#define XDNA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XDNA_ABI_VERSION 1

/* dtype codes */
#define XDNA_F32 0
#define XDNA_BF16 1
#define XDNA_F16 2
#define XDNA_I8 3
#define XDNA_U8 4
#define XDNA_I32 5

/* status codes (negative; positive values are hipError_t) */
#define XDNA_OK 0
#define XDNA_EINVAL (-1)
#define XDNA_EUNSUPPORTED (-2)
#define XDNA_ENODEV (-3)

/* GEMM / conv kinds of the tile table (xdna_tile_set). */
#define XDNA_KIND_I8 0   /* xdna_gemm_i8_i32 / xdna_gemm_i8_dequant: (m, n, k) as passed */
#define XDNA_KIND_BF16 1 /* xdna_gemm_bf16: (m, n, k) as passed (k in bf16 elements) */
#define XDNA_KIND_CONV 2 /* xdna_conv3x3_i8: m = nb * h * w, n = co, k = 9 * c_pad */

/* Tile ids: the tile engine's workgroup tiles (rows x columns of the output, waves), the small-M
 * (weight-streaming) kernel by waves per workgroup, the one-row (M = 1) kernel by waves per workgroup
 * (one output column per wave), the few-row (M <= 16) kernel by output columns per workgroup
 * (8 or 16), and tile-engine tiles whose workgroup splits K between 2 or 4 groups of waves (K2 / K4);
 * a tile forced on a shape its kernel does not take falls back to the built-in rule. */
#define XDNA_TILE_AUTO 0
#define XDNA_TILE_256x256W8 1
#define XDNA_TILE_256x256W4 2
#define XDNA_TILE_256x128 3
#define XDNA_TILE_128x256 4
#define XDNA_TILE_128x128 5
#define XDNA_TILE_64x64 6
#define XDNA_TILE_SMALL_W1 7
#define XDNA_TILE_SMALL_W2 8
#define XDNA_TILE_SMALL_W4 9
#define XDNA_TILE_SMALL_W8 10
#define XDNA_TILE_SMALL_W16 11
#define XDNA_TILE_192x256 12
#define XDNA_TILE_256x192 13
#define XDNA_TILE_64x32 14
#define XDNA_TILE_32x64 15
#define XDNA_TILE_32x32 16
#define XDNA_TILE_GEMV_W4 17
#define XDNA_TILE_GEMV_W2 18
#define XDNA_TILE_GEMV_W8 19
#define XDNA_TILE_SEG4_R2 20
#define XDNA_TILE_SEG4_R4 21
#define XDNA_TILE_64x64K2 22
#define XDNA_TILE_64x64K4 23
#define XDNA_TILE_32x64K4 24
#define XDNA_TILE_32x32K4 25
#define XDNA_TILE_128x128K2 26
#define XDNA_TILE_128x256W8 27
#define XDNA_TILE_256x128W8 28
#define XDNA_TILE_256x256PP 29  /* 256 x 256, 8 waves, ping-pong schedule (two groups of four waves) */
#define XDNA_TILE_256x64 30     /* 256 x 64, 4 waves stacked along M (narrow outputs with many rows) */
#define XDNA_TILE_DIRECT 31     /* convs only: register-operand kernels for c_pad 16..64, co a multiple of 32 <= 128 */

/* Library version (XDNA_ABI_VERSION). Replaces the import probe of kernels.available()
 * (torch_xdna/kernels.py:43-56): a loader checks it before trusting the other symbols. */
int xdna_abi_version(void);

/* Message of the last non-zero status returned on this thread ("" if none). The reference
 * surfaces launcher failures as Python exceptions caught at torch_xdna/runtime.py:294-295. */
const char* xdna_last_error(void);

/* Number of compute units and the gfx architecture of the current device, for launch shaping
 * and for reports (replaces kernels.unavailable_reason(), torch_xdna/kernels.py:59-60). */
int xdna_device_info(int* num_cus, int* gfx_major, int* gfx_minor);

/* Per-shape tile table (replaces the reference's tuned NPU tilings: kernels.tuned_table /
 * tiling_for, torch_xdna/kernels.py:123-149, filled from tools/sweep.py). xdna_tile_set makes
 * the first (head) launch of every later call of exactly (kind, m, n, k) use `tile`
 * (XDNA_TILE_AUTO removes the entry); any tile computes the same results, only the speed differs.
 * The table is process-wide and thread-safe. xdna_tile_get returns the head tile the next such call
 * uses (the table's, else the built-in rule's, which needs the current device) or a negative
 * status; xdna_tile_clear empties the table.
 *
 * A call whose head tile runs one workgroup per CU and whose last round of tiles would leave more
 * than half of the CUs idle runs rows [0, m1) with the head tile and rows [m1, m) as a second launch
 * with a smaller tail tile (the table's entry for (kind, m - m1, n, k) if it lists a tile-engine
 * tile, else the built-in rule's). xdna_tile_plan reports that whole plan of a call: *head, *m1 (0:
 * one launch, no tail) and *tail (XDNA_TILE_AUTO when there is none). GEMM operands above 1 GB run
 * in row chunks; the plan is then that of the first chunk. The reference's verify key names the
 * program of a launch (runtime.py:207: dtype, row bucket, Np, Kp, tiling); the plan is what
 * identifies the kernels of a call here. */
int xdna_tile_set(int kind, int64_t m, int64_t n, int64_t k, int tile);
int xdna_tile_get(int kind, int64_t m, int64_t n, int64_t k);
int xdna_tile_plan(int kind, int64_t m, int64_t n, int64_t k, int* head, int64_t* m1, int* tail);
int xdna_tile_clear(void);

/* Per-row symmetric int8 quantization of activations or weights:
 *   s[r] = max(amax_k |x[r,k]|, 1e-8f) / 127  (IEEE float32 division),
 *   q[r,k] = clamp(round_half_even(x[r,k] / s[r]), -127, 127),
 * bit-exact with torch_xdna/runtime.py:145-148 (`_quant_rows`), :366-368 (`linear_int8`) and
 * :64-65 (`QWeight`). x is [rows, k] of x_dtype (XDNA_F32/BF16/F16) with row stride ld_x; q is
 * written as [rows, k_pad] with row stride ld_q, columns [k, k_pad) set to 0; s is [rows]. */
int xdna_quant_rows(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ld_x, int8_t* q,
                    int64_t ld_q, int64_t k_pad, float* s, void* stream);

/* c[m, n] = sum_k a[m, k] * w[n, k] in exact int32 (int8 x int8 -> int32).
 * Replaces kernels.mm_i8 + matmul_i8_k (torch_xdna/kernels.py:172-192,
 * torch_xdna/_triton_kernels.py:6-23) behind runtime._npu_acc (torch_xdna/runtime.py:191-209);
 * bit-exact with torch._int_mm(xq, w_kn) (torch_xdna/runtime.py:162-163). No padding of M or N
 * is needed; k % 16 == 0, lda and ldw multiples of 16, ldc >= n. */
int xdna_gemm_i8_i32(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int32_t* c,
                     int64_t ldc, int64_t m, int64_t n, int64_t k, void* stream);

/* The W8A8 linear with its dequantize fused into the GEMM epilogue:
 *   y[m, n] = ((float)acc[m, n] * sx[m]) * sw[n] (+ bias[n]) in float32, each step rounded
 *   once, then converted to y_dtype (XDNA_F32/BF16/F16, round to nearest even),
 * the arithmetic of torch_xdna/runtime.py:350-353 / :429-432 (`linear`, `linear_cat`) and
 * :370-374 (`linear_int8`). bias may be NULL. Same operand rules as xdna_gemm_i8_i32. */
int xdna_gemm_i8_dequant(const int8_t* a, int64_t lda, const float* sx, const int8_t* w, int64_t ldw,
                         const float* sw, const float* bias, void* y, int y_dtype, int64_t ldy,
                         int64_t m, int64_t n, int64_t k, void* stream);

/* xdna_gemm_i8_i32 and xdna_gemm_i8_dequant with a workspace, for shapes whose tiles (up to 64 x 64)
 * would leave most of the GPU idle (decode-sized M against N of a few thousand, short-M GEMMs): the
 * workgroups of a tile split its K, each stores its int32 partial sums in ws, and the last to finish
 * adds the others' and runs the epilogue. Results are identical to the calls without a workspace
 * (integer sums are exact in any order); the replaced reference interfaces are theirs
 * (torch_xdna/kernels.py:172-192 and torch_xdna/runtime.py:350-353 / :429-432 / :370-374).
 * ws: 256-byte aligned device memory whose first XDNA_GEMM_WS_COUNTER_BYTES are zero before its first
 * use (every call leaves them zero); the rest is overwritten. A launch splits only where ws_bytes
 * holds its split, so any size (or NULL) is valid; xdna_gemm_ws_bytes(m, n, k) gives the size that
 * allows every split a call of that shape makes (0: it makes none). Calls that share a workspace must
 * be ordered (one stream): concurrent calls on one workspace race. */
#define XDNA_GEMM_WS_COUNTER_BYTES 65536
int64_t xdna_gemm_ws_bytes(int64_t m, int64_t n, int64_t k);
/* The K split of a call's launches with a workspace of xdna_gemm_ws_bytes (for the first row chunk:
 * *head_ks for rows [0, m1) of xdna_tile_plan, *tail_ks for the tail; 1: no split). Part of the launch
 * plan a per-kernel-variant verify cache keys on (the reference's `_verified` key, runtime.py:207). */
int xdna_gemm_ksplit(int64_t m, int64_t n, int64_t k, int* head_ks, int* tail_ks);
int xdna_gemm_i8_i32_ws(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int32_t* c,
                        int64_t ldc, int64_t m, int64_t n, int64_t k, void* ws, int64_t ws_bytes,
                        void* stream);
int xdna_gemm_i8_dequant_ws(const int8_t* a, int64_t lda, const float* sx, const int8_t* w, int64_t ldw,
                            const float* sw, const float* bias, void* y, int y_dtype, int64_t ldy,
                            int64_t m, int64_t n, int64_t k, void* ws, int64_t ws_bytes, void* stream);

/* The W8A8 linear of ONE activation row (decode, M = 1) in one launch: the row's per-row quantize
 * (xdna_quant_rows' arithmetic, replacing torch_xdna/runtime.py:287 `_quant_rows` in `_gemm` and
 * :145-148) and the GEMM with the dequantize of xdna_gemm_i8_dequant (runtime.py:288-296 and :350-353,
 * `linear` / `linear_cat` at one row), so
 *   y[n] = ((float)sum_k q[k] * w[n, k] * s) * sw[n] (+ bias[n]),  s = max(max_k |x[k]|, 1e-8f) / 127,
 *   q[k] = clamp(round_half_even(x[k] / s), -127, 127),
 * bit for bit what xdna_quant_rows followed by xdna_gemm_i8_dequant computes. x: kx elements of
 * x_dtype (XDNA_F32/BF16/F16), 16-byte aligned, kx * element size a multiple of 16 bytes; the
 * elements [kx, k) count as zeros. w: [n, k] int8 with row stride ldw (k % 16 == 0,
 * 16 <= k <= XDNA_LINEAR_ROW_KMAX). y: n elements of y_dtype. sx: NULL, or where the row's scale s
 * is written (when n > 0). No workspace. */
#define XDNA_LINEAR_ROW_KMAX 32768
int xdna_linear_row(const void* x, int x_dtype, int64_t kx, const int8_t* w, int64_t ldw, const float* sw,
                    const float* bias, void* y, int y_dtype, int64_t n, int64_t k, float* sx, void* stream);

/* The bf16 GEMM of precision "bf16": y[m, n] = sum_k a[m, k] * w[n, k] with bf16 operands and float32
 * accumulation (+ bias[n] in float32), converted to y_dtype (XDNA_F32/BF16/F16, round to nearest
 * even). Replaces kernels.mm_bf16 (torch_xdna/kernels.py:167-169) behind runtime._npu_bf16 /
 * _gemm_bf16 (torch_xdna/runtime.py:212-237, :299-313) with the bf16 weight copy of
 * QWeight.npu_bf16 (:80-86). Float sums are not bit-exact across summation orders: the result is
 * the float32 sum of the exact bf16 products to within K float32 roundings (the reference checks
 * its NPU to a 5e-2 relative norm, runtime.py:179-182). a: [m, k] bf16, row stride lda; w: [n, k]
 * bf16, row stride ldw; k % 8 == 0 (zero-pad), lda and ldw multiples of 8, 16-byte aligned; bias
 * may be NULL. */
int xdna_gemm_bf16(const void* a, int64_t lda, const void* w, int64_t ldw, const float* bias, void* y, int y_dtype,
                   int64_t ldy, int64_t m, int64_t n, int64_t k, void* stream);

/* dst[r, :cols] = src[r, :cols], dst[r, cols:cols_pad] = 0 for int8 rows (aligning an int8
 * activation handed to xdna::linear_i8, torch_xdna/ops.py:49-55, to the 16-byte K rule). */
int xdna_pad_rows_i8(const int8_t* src, int64_t rows, int64_t cols, int64_t ld_src, int8_t* dst,
                     int64_t ld_dst, int64_t cols_pad, void* stream);

/* Floats of caller scratch per image for the per-image max of the two calls below (block maxima,
 * reduced by the kernel that needs the image's max: no atomics, nothing to clear first). */
#define XDNA_AMAX_WS_PER_IMAGE 256

/* Per-image quantization of an NCHW activation into the conv's NHWC int8 layout:
 *   sx[b] = max(amax |x[b]|, 1e-8f) / 127 over the whole image (C*H*W values),
 *   q[b, p, c] = clamp(round_half_even(x[b, c, p] / sx[b]), -127, 127) for c < ch, 0 for
 *   ch <= c < c_pad, p = y * w + x,
 * bit-exact with torch_xdna/conv.py:45-46 (`conv3x3_int8`). amax_ws is caller scratch of
 * nb * XDNA_AMAX_WS_PER_IMAGE floats (overwritten). */
int xdna_conv_quant_nhwc(const void* x, int x_dtype, int64_t nb, int64_t ch, int64_t h, int64_t w,
                         int8_t* q, int64_t c_pad, float* sx, float* amax_ws, void* stream);

/* xdna_conv_quant_nhwc without the caller workspace, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in
 * the reference. The per-image block maxima go to a file-scope device array of the library
 * (XDNA_NOALLOC_MAX_IMAGES x XDNA_AMAX_WS_PER_IMAGE floats, 1 MB, held on each device until the process
 * ends; its address is looked up once per device on the first call). nb above XDNA_NOALLOC_MAX_IMAGES is
 * rejected (XDNA_EINVAL). Every call on a device shares that array: calls that overlap on one device
 * (other streams, other threads) race and must be serialized by the caller. Nothing is allocated: no
 * hipMalloc / hipFree. Same results as xdna_conv_quant_nhwc. */
#define XDNA_NOALLOC_MAX_IMAGES 1024
int xdna_conv_quant_nhwc_noalloc(const void* x, int x_dtype, int64_t nb, int64_t ch, int64_t h, int64_t w, int8_t* q,
                                 int64_t c_pad, float* sx, void* stream);

/* Conv weight quantize-once (torch_xdna/conv.py:58-60, `ConvLayer.__init__`):
 *   sw[o] = max(amax |w[o]|, 1e-8f) / 127 over (Ci, 3, 3); wq = clamp(round(w / sw), +-127),
 * written in the kernel's layout wq[o][ky*3+kx][c] with ci_pad channels (zeros past ci).
 * w is [co][ci][3][3] of w_dtype. */
int xdna_conv_weight_pack(const void* w, int w_dtype, int64_t co, int64_t ci, int8_t* wq, int64_t ci_pad,
                          float* sw, void* stream);

/* int8 3x3 / stride 1 / padding 1 convolution as an implicit GEMM on MFMA, with the requantize of
 * torch_xdna/conv.py:89-92 fused: q = sat((acc + (1 << (shift-1))) >> shift) to [0, 255] (uint8)
 * when relu, else [-128, 127] (int8). Replaces Triton-XDNA's Conv3x3 launch
 * (torch_xdna/conv.py:78-84, :94-96; kernel math npu_kernels/conv3x3_cascade.cc:24-131).
 * x: NHWC [nb, h, w, c_pad] int8; wq: [co][9][c_pad]; y: NHWC [nb, h, w, co] (int8 or uint8).
 * If acc_max is not NULL the launch is a calibration pass (torch_xdna/conv.py:71-75): nothing is
 * written to y (which may be NULL), shift is ignored, and acc_max[0] receives max(acc, 0) when
 * relu else max |acc| over all outputs. c_pad % 16 == 0, 1 <= shift <= 31. */
int xdna_conv3x3_i8(const int8_t* x, int64_t nb, int64_t h, int64_t w, int64_t c_pad, const int8_t* wq,
                    int64_t co, int shift, int relu, void* y, int32_t* acc_max, void* stream);

/* Conv dequantize back to NCHW (torch_xdna/conv.py:48-51):
 *   y[b, o, p] = (float)q[b, p, o] * (scale[o] * sx[b]) (+ bias[o]) -> y_dtype,
 * q NHWC [nb, h*w, co] int8 (uint8 when relu). bias may be NULL. */
int xdna_conv_dequant(const void* q, int relu, int64_t nb, int64_t h, int64_t w, int64_t co,
                      const float* scale, const float* sx, const float* bias, void* y, int y_dtype,
                      void* stream);

/* The conv, its requantize and the dequantize in one launch: what xdna_conv3x3_i8 followed by
 * xdna_conv_dequant computes (the GPU form of conv3x3_int8's conv + dequant, torch_xdna/conv.py:47-51),
 * bit for bit, without the NHWC integers in memory. x NHWC [nb, h, w, c_pad] int8, wq [co][9][c_pad],
 * scale [co] (the weight scales), sx [nb] (the per-image input scales), bias [co] or NULL;
 * y NCHW [nb, co, h, w] of y_dtype (XDNA_F32/BF16/F16), 16-byte aligned. 1 <= shift <= 31. */
int xdna_conv3x3_dequant(const int8_t* x, int64_t nb, int64_t h, int64_t w, int64_t c_pad, const int8_t* wq,
                         int64_t co, int shift, int relu, const float* scale, const float* sx, const float* bias,
                         void* y, int y_dtype, void* stream);

/* Conv-to-conv chaining (the reference's "What is left", results/conv3x3_cascade.md:216-222): the
 * previous conv's NHWC output q [nb, h, w, co] (uint8 when relu) goes straight to the next conv's
 * NHWC int8 input xq_next [nb, h', w', c_pad_next] with its per-image scale sx_next [nb], computing
 * exactly what the reference's chain computes through float tensors: the dequantize of
 * torch_xdna/conv.py:48-50 (q * (scale[o] * sx[b]) (+ bias[o]), cast to x_dtype), the 2x2 / stride-2
 * max-pool between the layers when pool != 0 (h' = h / 2, w' = w / 2), and the next layer's
 * per-image quantize (conv.py:45-46). relu_y != 0 adds the graph ReLU that follows a biased conv
 * (torch_xdna/backend.py:161-165 fuses a ReLU only into bias-free convs). Pooling runs on the
 * integers (the dequantize is non-decreasing in q). amax_ws is caller scratch of
 * nb * XDNA_AMAX_WS_PER_IMAGE floats (overwritten). */
int xdna_conv_requant_next(const void* q, int relu, int relu_y, int pool, int64_t nb, int64_t h, int64_t w, int64_t co,
                           const float* scale, const float* sx, const float* bias, int x_dtype, int8_t* xq_next,
                           int64_t c_pad_next, float* sx_next, float* amax_ws, void* stream);

/* int8 layout changes for the reference op's NCHW int8 contract (torch_xdna/ops.py:64-76):
 * NCHW [nb, ch, h, w] -> NHWC [nb, h, w, c_pad] (zero channels past ch), and
 * NHWC [nb, h, w, ch] -> NCHW [nb, ch, h, w] (one byte per element, int8 or uint8). */
int xdna_nchw_to_nhwc_i8(const int8_t* src, int64_t nb, int64_t ch, int64_t h, int64_t w, int8_t* dst,
                         int64_t c_pad, void* stream);
int xdna_nhwc_to_nchw_i8(const void* src, int64_t nb, int64_t ch, int64_t h, int64_t w, void* dst,
                         void* stream);

/* ---- xdna::qwen3_stack (replaces Triton-XDNA's tl.extra.npu.qwen3_stack, called from
 * torch_xdna/stack.py:360-390 `run`). The stack runs on a packed activation of T valid tokens
 * (all sequences one after another); its GEMMs are xdna_gemm_bf16 calls. Transformers' Qwen3
 * semantics (modeling_qwen3: Qwen3RMSNorm, Qwen3Attention with q_norm / k_norm and RoPE,
 * Qwen3MLP). */

/* y[r, :] = bf16(w * (x[r, :] * rsqrt(mean(x[r, :]^2) + eps))), x float32 [rows, d], w [d] of
 * w_dtype; d a multiple of 256, at most 4096. */
int xdna_rmsnorm_bf16(const float* x, int64_t rows, int64_t d, const void* w, int w_dtype, float eps, void* y,
                      void* stream);

/* qkv float32 [T, (nh + 2 nkv) * 128] (q heads, then k heads, then v heads; head_dim 128): q and k
 * heads RMSNorm'd over the head with q_w / k_w [128], then RoPE at position pos[t]
 * (theta_j = pos * inv_freq[j], j < 64, rotate_half pairing j with j + 64), written bf16 to
 * q [T, nh, 128] and k [T, nkv, 128]; v heads written bf16 transposed to vt[kv head][dim][vt_col[t]]
 * (row stride ld_vt). */
int xdna_qk_norm_rope(const float* qkv, int64_t T, int nh, int nkv, const void* q_w, const void* k_w, int w_dtype,
                      const float* inv_freq, const int32_t* pos, const int32_t* vt_col, float eps, void* q, void* k,
                      void* vt, int64_t ld_vt, void* stream);

/* Bidirectional attention per sequence s (tokens seq_start[s] .. + seq_len[s] of q / k, vt columns
 * seq_vt[s] .. + round_up(seq_len[s], 32), zero past seq_len[s]) and q head h (kv head
 * h / (nh / nkv)): out = softmax(q k^T * scale) v, bf16 [T, nh, 128]. max_len >= every seq_len;
 * ld_vt and seq_vt multiples of 8. */
int xdna_attention_bf16(const void* q, const void* k, const void* vt, int64_t ld_vt, const int32_t* seq_start,
                        const int32_t* seq_len, const int32_t* seq_vt, int64_t nseq, int64_t max_len, int nh, int nkv,
                        float scale, void* out, void* stream);

/* y = bf16(silu(gu[:, :inter]) * gu[:, inter:]), gu float32 [T, 2 inter] (gate, then up). */
int xdna_silu_mul_bf16(const float* gu, int64_t T, int64_t inter, void* y, void* stream);

/* The gate|up projection of Qwen3MLP with `act_fn(gate_proj(x)) * up_proj(x)` fused into the GEMM:
 * y[m, c] = bf16(silu(g) * u), g and u the float32 sums of a[m, :] with gate row c and up row c
 * (silu(g) = g / (1 + exp(-g))), the values of xdna_gemm_bf16 (float32 out) then xdna_silu_mul_bf16
 * in one launch. w is [n2, k] bf16 with the gate and up rows interleaved in pairs: rows 4j, 4j + 1 are
 * gate rows 2j, 2j + 1 and rows 4j + 2, 4j + 3 up rows 2j, 2j + 1 (n2 = 2 inter, a multiple of 4); y is
 * bf16 [m, n2 / 2] with row stride ldy (even, 4-byte aligned). Operand rules of xdna_gemm_bf16. */
int xdna_gemm_bf16_silu(const void* a, int64_t lda, const void* w, int64_t ldw, void* y, int64_t ldy, int64_t m,
                        int64_t n2, int64_t k, void* stream);

/* x += y over n float32 values (residual adds). */
int xdna_add_f32(float* x, const float* y, int64_t n, void* stream);

/* The residual add and the RMSNorm that follows it in a Qwen3 layer (Qwen3DecoderLayer's
 * `hidden_states = residual + hidden_states` then the next Qwen3RMSNorm) in one launch: x += a (float32,
 * x and a [rows, d]), then y as xdna_rmsnorm_bf16 of the updated x. The same values as
 * xdna_add_f32 followed by xdna_rmsnorm_bf16. */
int xdna_add_rmsnorm_bf16(float* x, const float* a, int64_t rows, int64_t d, const void* w, int w_dtype, float eps,
                          void* y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* XDNA_HIP_H */
