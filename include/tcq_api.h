/* C ABI of the MI355X (gfx950) TCQ W2A8 deploy path: trellis-coded 2-bit weights (bitshift trellis L = 16, K = 2, V = 2,
 * 16 x 16 tiles, 512 x 2 table per layer, per-row scales, two-sided randomized block-Walsh rotation) with 8-bit per-token
 * activations, and the W8A8 INT8 GEMM.
 *
 * Every entry point takes device pointers, sizes and a stream (a hipStream_t passed as void*; NULL = the default stream),
 * launches asynchronously on that stream, allocates nothing and copies nothing between host and device, so calls can be
 * captured into HIP graphs. Return value: TCQ_OK, a negative TCQ_ERR_* for an argument the call rejects before launching, or
 * a positive hipError_t reported by the launch.
 *
 * Each declaration names the reference interface it replaces (paths relative to the reference repository). The reference
 * launched NVRTC-compiled CUDA kernels through ctypes (deploy/tcq_kernels/cuda_rt.py:87-108) from Python helpers with
 * caller-allocated outputs (deploy/tcq_kernels/kernels.py:602-696); these functions are that boundary as a C ABI.
 *
 * Layouts (all row-major, C order):
 *   bits       (m/16 * n/16, 32) uint16: the packed stream, 32 words per tile, tiles row-major (tcq_format.py:3-4)
 *   wdev       device layout of the same words made by tcq_repack (see there); required by the fused products
 *   tlut       (512, 2) FP16 table; t8: (512, 2) INT8 table (tcq_format.py:74-77)
 *   row_scale  (m,) FP16; rs: (m,) FP32; su: (n,) int8 +-1; sv: (m,) int8 +-1
 *   q          (M, K) int8 row-major; q4: (K/4, ldq) int32, 4 consecutive inputs per word, token = column, or with
 *              ldq == TCQ_LDQ_TOKEN_BLOCKS the token-block layout (16-byte aligned, K % 16 == 0; defined below)
 */
#ifndef TCQ_API_H
#define TCQ_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* tcq_stream_t;

enum tcq_status {
    TCQ_OK = 0,
    TCQ_ERR_ARG = -1,         /* null pointer where one is required, or a non-positive size */
    TCQ_ERR_SHAPE = -2,       /* sizes violate the format (m, n multiples of 16; K multiple of 4; widths too large) */
    TCQ_ERR_DTYPE = -3,       /* unsupported dtype code for this entry point */
    TCQ_ERR_UNSUPPORTED = -4, /* a size the kernel has no variant for (e.g. more tokens than the small-M products take) */
    TCQ_ERR_ALIGN = -5        /* a pointer the kernel reads or writes in 16-byte vectors is not 16-byte aligned */
};

enum tcq_dtype { TCQ_F32 = 0, TCQ_BF16 = 1, TCQ_F16 = 2, TCQ_I32 = 3, TCQ_I8 = 4 };

/* Token-block layout of INT8 activations (M tokens, K columns, K % 16 == 0): token t, column k at byte
 * ((t / 16 * K / 16 + k / 16) * 16 + t % 16) * 16 + k % 16, in a buffer of ceil(M / 16) * 16 * K bytes. 16 columns of 16
 * tokens form a contiguous 256-byte group, so the small-M products read every activation fragment of 16 tokens x 64
 * columns as one contiguous KiB (row-major rows make it 16 separate 64-byte pieces). No reference counterpart: it plays the
 * part of the reference's q4 layout (kernels.py:170-184), the layout the reference's small-M kernels read.
 * The quantizing entry points write it through their q4 output when ldq == TCQ_LDQ_TOKEN_BLOCKS; tcq_gemm_tcq and
 * tcq_gemm_w8 read q in it when out_dtype carries TCQ_Q_TOKEN_BLOCKS. */
#define TCQ_LDQ_TOKEN_BLOCKS (-16)
#define TCQ_Q_TOKEN_BLOCKS 0x100

/* K parts: the int32 sums of a small-M product split over P = 2 or 4 consecutive ranges of its 256-column K chunks (chunks
 * [p * ceil(nch / P), ...) for part p), each written whole, part p at out + p * M * ldo elements. Flag of out_dtype
 * (with TCQ_I32) for tcq_gemm_tcq / tcq_gemm_w8, and of acc_dtype (with TCQ_I32) for tcq_post_add_norm_pre, which adds the
 * P parts (exact int32; part p at acc + p * M * lda) before scaling. A product of few tile rows then spreads over P times
 * as many workgroups, and the consumer reads P partial rows instead of one. No reference counterpart (the reference's
 * small-M products cover K in one block, kernels.py:365-427). */
#define TCQ_K_PARTS2 0x200
#define TCQ_K_PARTS4 0x400

/* Stage-split gated-MLP input (flag of out_dtype, with TCQ_F32, for tcq_gemm_tcq at M <= 16, K <= 4096, every segment m a
 * multiple of 128): each segment's FP32 z = (float(acc) s) rs goes through the first seven stages of its block Walsh
 * (h = 1 .. 64, which stay inside blocks of 128 rows, in the reference's stage order) inside the product, and is stored
 * block-transposed, out (M, 128, m / 128): row 128 b + o of token t at out[(t * 128 + o) * (m / 128) + b]. tcq_glu_split
 * finishes the middle from it. No reference counterpart: it splits tcq_mid2 (kernels.py:263-278) over many CUs. */
#define TCQ_Z_W128T 0x1000

/* One-token products on v_dot4c_i32_i8 (flag of out_dtype for tcq_gemm_tcq / tcq_gemm_w8, M == 1 only): each lane
 * multiplies its 16 weights of a tile row with the token's 16 activations in four 4-byte dot products instead of
 * a 16 x 16 x 64 MFMA whose 15 other token columns are zero; the sums are the same exact int32 values. Every plan and
 * every other flag keeps its meaning. The reference's one-token products are dot products (__dp4a, kernels.py:365-382). */
#define TCQ_DOT4 0x2000

/* Library version string and the widest row the block-Walsh kernels take (16384). */
const char* tcq_version(void);
int tcq_max_width(void);

/* ---------------------------------------------------------------------------------------------------------- load time */

/* INT8 table and row scale of one layer: t8 = clamp(round(tlut * g), +-127), g = float(1/max|tlut|) * 127,
 * rs = float(row_scale) / g; gain (1 float, may be NULL) receives g.
 * Replaces tcq_format.snap (deploy/tcq_kernels/tcq_format.py:74-77), called by tcq_format.Layer.__init__ (:90). */
int tcq_snap(const void* tlut, const void* row_scale, int m, int8_t* t8, float* rs, float* gain, tcq_stream_t stream);

/* Row-group tables (the GR00T variants, baselines/groot/simpler/main_row/scripts/groot_tcq.py:154-175): tlut (G, 512, 2), rows
 * split evenly into G contiguous groups (row i reads table i / (m / G)). Each table snaps on its own: t8 (G, 512, 2), gain
 * (G,), rs[i] = row_scale[i] / gain[group of i]. m % G == 0. No reference counterpart for the INT8 snap of grouped tables:
 * it is tcq_format.snap applied per group. */
int tcq_snap_groups(const void* tlut, int G, const void* row_scale, int m, int8_t* t8, float* rs, float* gain, tcq_stream_t stream);

/* Reference word layout -> device layout for the fused products (tcq_gemv_f16, tcq_gemm_tcq). For tile row I and chunk c of
 * 16 tiles (columns 256 c .. 256 c + 255) the device layout holds 1 KiB: dword 4 l + j of lane l = 16 g + r is the 32-bit
 * window (word[2r] << 16) | word[2r + 1] of tile 16 c + 4 j + g. n is padded to a multiple of 256 with zero words.
 * wdev holds (m/16) * ceil(n/256) * 256 uint32. No reference counterpart: the reference streams the words as stored
 * (kernels.py:403-427); this is a load-time permutation of the same 2 bits per weight. */
int tcq_repack(const void* bits, void* wdev, int m, int n, tcq_stream_t stream);
int64_t tcq_repack_words(int m, int n);

/* ------------------------------------------------------------------------------------------------------------- decode */

/* Dense INT8 decode: out (m, n) int8 = sign * t8[hash(state)]. Replaces kernels.decode / k_decode
 * (deploy/tcq_kernels/kernels.py:339-349, 653-656); definition tcq_format.Layer.w8_reference (tcq_format.py:97-98). */
int tcq_decode_i8(const void* bits, const int8_t* t8, int8_t* out, int m, int n, tcq_stream_t stream);
/* The same from the tcq_repack words of the layer (one table, t8 (512, 2)): the bytes of tcq_decode_i8, read through the
 * coalesced layout of the fused products (the prefill of a runtime that keeps the repacked words). words and out 16-byte
 * aligned. No reference counterpart beyond kernels.decode. */
int tcq_decode_i8_words(const void* words, const int8_t* t8, int8_t* out, int m, int n, tcq_stream_t stream);
/* The same with G row-group tables t8 (G, 512, 2); (m / G) % 16 == 0. */
int tcq_decode_i8_groups(const void* bits, const int8_t* t8, int G, int8_t* out, int m, int n, tcq_stream_t stream);

/* Dense decode through a 16-bit table: out (m, n) = sign * tlut[hash(state)], the sign flipping bit 15 of the first
 * coordinate (exact for FP16 and BF16 tables). With the FP16 table: tcq_format.lookup(states, tlut.float())
 * (tcq_format.py:66-71, 103, 139); with the BF16 bit patterns of the INT8 table values: kernels.decode_bf16 / k_decode_bf16
 * (kernels.py:320-337, 683-686). */
int tcq_decode_f16(const void* bits, const void* tlut, void* out, int m, int n, tcq_stream_t stream);
/* The same with G row-group tables (G, 512, 2) (groot_tcq.py:165-175 decode_normalized); (m / G) % 16 == 0. */
int tcq_decode_f16_groups(const void* bits, const void* tlut, int G, void* out, int m, int n, tcq_stream_t stream);

/* ----------------------------------------------------------------------------------------------------------- rotation */

/* Randomized block-Walsh transform of M rows: y = fwht(x * su) (su may be NULL: no sign flip), FP32 butterflies in stage
 * order h = 1, 2, 4, ..., normalised per power-of-two block. x_dtype in {F32, BF16, F16}, y_dtype in {F32, BF16, F16}.
 * Leading dimensions in elements. Replaces tcq_format.fwht (deploy/tcq_kernels/tcq_format.py:44-55) applied to x * su
 * (tcq_format.py:130). */
int tcq_rht(const void* x, int x_dtype, int ldx, const int8_t* su, void* y, int y_dtype, int ldy, int M, int n,
            tcq_stream_t stream);

/* Rotate + quantize: sign, block Walsh, per-token absmax, INT8. q (M, K) row-major and / or q4 (K/4, ldq) int32 (either may
 * be NULL), scale (M,) FP32. Replaces kernels.pre / k_pre_bf16 / k_pre_f32 (deploy/tcq_kernels/kernels.py:208-219, 602-606);
 * definition quantize_tokens(fwht(x * su)) (tcq_format.py:119-122, 130-134). */
int tcq_pre(const void* x, int x_dtype, const int8_t* su, int8_t* q, int32_t* q4, int ldq, float* scale, int M, int K,
            tcq_stream_t stream);

/* tcq_pre with FP16 column scales col_scale (K,) applied to the rotated activations before the absmax and the INT8 rounding:
 * q, scale of quantize_tokens(fwht(x * su) * col_scale) (col_scale NULL: tcq_pre). The column scale of the GR00T row-group
 * records (baselines/groot/simpler/main_row/scripts/groot_tcq.py:178-184: W = S_v H_m diag(r) Q diag(c) H_n S_u, c in the
 * rotated input basis) moves onto the activations this way; the reference deploy path has no column scale. */
int tcq_pre_cs(const void* x, int x_dtype, const int8_t* su, const void* col_scale, int8_t* q, int32_t* q4, int ldq, float* scale,
               int M, int K, tcq_stream_t stream);

/* Rotate for the float (W2) path: h16 (M, K) FP16 = fwht(x * su) / hscale[t], hscale[t] (M,) FP32 a power of two that puts
 * the row's absmax in [2^14, 2^15) (1 for a zero row), so the division is exact and FP16 cannot overflow. Counterpart of
 * kernels.pre_h (kernels.py:309-317, 677-680), which rounds to BF16 instead. */
int tcq_pre_h16(const void* x, int x_dtype, const int8_t* su, void* h16, float* hscale, int M, int K, tcq_stream_t stream);

/* Per-row symmetric INT8 without rotation (tcq_format.quantize_tokens, tcq_format.py:119-122): activations per token, or a
 * dense weight per output channel. q (M, K) int8, scale (M,) FP32. */
int tcq_quantize_rows(const void* x, int x_dtype, int ldx, int8_t* q, float* scale, int M, int K, tcq_stream_t stream);

/* Scale + rotate epilogue: z = SCALE(acc[t, col0 + i]) -> block Walsh -> * sv -> + bias -> y (M, N). sv NULL: a one-sided
 * layer (the GR00T "tcq" base, groot_tcq.py:187-191: W = Q H_n S_u, no output rotation): y = SCALE(acc) (+ bias).
 * acc_dtype I32: SCALE = (float(a) * s[t]) * rs[i]; F32: SCALE = a (s, rs ignored); BF16: SCALE = bf16(a) * rs[i].
 * bias FP32 (N,) or NULL. y_dtype in {BF16, F16, F32}. lda = leading dimension of acc in elements.
 * Replaces kernels.post / k_post_{i32,f32,bf16} (deploy/tcq_kernels/kernels.py:221-230, 545, 612-615). */
int tcq_post(const void* acc, int acc_dtype, int lda, int col0, const float* s, const float* rs, const int8_t* sv,
             const float* bias, void* y, int y_dtype, int M, int N, tcq_stream_t stream);

/* Most segments (layers) a by-value descriptor pack holds: tcq_post_group, tcq_gemm_tcq, tcq_gemm_w8. */
#define TCQ_MAX_SEGS 4

/* One segment of a batched epilogue: columns col0 .. col0 + N of M accumulator rows (stride lda elements) -> y (M, N). */
typedef struct tcq_post_seg {
    const void* acc;     /* accumulator base */
    const float* rs;     /* (N,) FP32 row scale (I32 / BF16 accumulators), else NULL */
    const int8_t* sv;    /* (N,) output signs */
    const float* bias;   /* (N,) FP32 or NULL */
    void* y;             /* (M, N) output, row stride N */
    int lda, col0, N;
    int gelu;            /* nonzero: BF16 output goes through the GELU table (gelu_lut must then be given) */
} tcq_post_seg;

/* Batched epilogue: one workgroup per (token, segment), each segment as tcq_post with its own columns, row scale, signs, bias,
 * output and optional GELU. segs is a DEVICE array of nseg descriptors; every segment's N must be <= maxN (a segment with
 * N > maxN or N <= 0 is skipped). acc_dtype and y_dtype apply to all segments; s (M,) FP32 per-token scales for I32
 * accumulators. gelu_lut: 65536 BF16 values, GELU (tanh) of every BF16 bit pattern, or NULL.
 * Replaces kernels.post3 / k_post3_* and kernels.postg / k_postg_* (deploy/tcq_kernels/kernels.py:232-261, 618-628), which
 * hold at most three segments sharing one accumulator row; here the count is free and each segment may have its own base. */
int tcq_postg(const tcq_post_seg* segs, int nseg, int acc_dtype, const float* s, const uint16_t* gelu_lut, int y_dtype, int M,
              int maxN, tcq_stream_t stream);

/* The epilogue of one layer group (q / k / v, gate / up: at most TCQ_MAX_SEGS layers), as tcq_postg, with segs a HOST array
 * copied into the launch: no device descriptor array, so every call may name new output buffers, also under HIP-graph
 * capture. A segment with gelu set needs gelu_lut and a BF16 output.
 * Replaces kernels.post3 / kernels.postg as Group.posts calls them (deploy/tcq_kernels/kernels.py:232-261, 618-628;
 * modules.py:95-106). */
int tcq_post_group(const tcq_post_seg* segs, int nseg, int acc_dtype, const float* s, const uint16_t* gelu_lut, int y_dtype,
                   int M, tcq_stream_t stream);

/* kernels.post3 / k_post3_{i32,f32,bf16} (deploy/tcq_kernels/kernels.py:232-247, 618-621), argument for argument: the three
 * layers of a q / k / v group read accumulator columns side by side (layer i from column n0 + ... + n(i-1) of each row of
 * stride lda); rs, sv and bias are the (n0 + n1 + n2,) concatenations (rs NULL for an F32 accumulator, bias may be NULL);
 * y0, y1, y2 (M, n_i) BF16. Same arithmetic as tcq_post per layer. */
int tcq_post3(const void* acc, int acc_dtype, const float* s, const float* rs, const int8_t* sv, const float* bias, void* y0,
              void* y1, void* y2, int M, int n0, int n1, int n2, int lda, tcq_stream_t stream);
/* kernels.postg / k_postg_* (deploy/tcq_kernels/kernels.py:249-261, 624-628), argument for argument: two or three layers
 * (n2 <= 0 and y2 NULL for two) as tcq_post3, one workgroup per (token, layer); gelu0 nonzero sends the first layer's BF16
 * output through gelu_lut (65536 BF16 values, required then). */
int tcq_postg3(const void* acc, int acc_dtype, const float* s, const float* rs, const int8_t* sv, const float* bias,
               const uint16_t* gelu_lut, void* y0, void* y1, void* y2, int M, int n0, int n1, int n2, int lda, int gelu0,
               tcq_stream_t stream);

/* ----------------------------------------------------------------------------------------------------- MLP middles */

/* Gated-MLP middle (down(gelu(gate(x)) * up(x))): acc (M, lda >= 2N) holds gate columns [0, N) and up columns [N, 2N),
 * scaled as tcq_post (rs, sv: concatenated (2N,) vectors; rs unused for F32). g = GELU(BF16(walsh(gate) * sv)) by the table,
 * u = BF16(walsh(up) * sv), x = BF16(g * u) * su (su: the down projection's input signs, (N,)) -> block Walsh -> per-token
 * INT8: q (M, N) and / or q4 (N/4, ldq), scale (M,). N % 16 == 0, N <= tcq_max_width().
 * Replaces kernels.mid2 / k_mid2_{i32,f32,bf16} (deploy/tcq_kernels/kernels.py:263-278, 640-643). */
int tcq_mid2(const void* acc, int acc_dtype, int lda, const float* s, const float* rs, const int8_t* sv, const uint16_t* gelu_lut,
             const int8_t* su, int8_t* q, int32_t* q4, int ldq, float* scale, int M, int N, tcq_stream_t stream);

/* Plain-MLP middle (fc2(gelu(fc1(x)))): acc (M, lda >= N) -> walsh -> * sv -> + bias (FP32 (N,) or NULL) -> BF16 -> GELU table
 * -> * su -> walsh -> per-token INT8 (q / q4, scale); N % 16 == 0. Replaces kernels.mid1 / k_mid1_* (deploy/tcq_kernels/kernels.py:280-292,
 * 646-650). */
int tcq_mid1(const void* acc, int acc_dtype, int lda, const float* s, const float* rs, const int8_t* sv, const float* bias,
             const uint16_t* gelu_lut, const int8_t* su, int8_t* q, int32_t* q4, int ldq, float* scale, int M, int N,
             tcq_stream_t stream);

/* Second half of a split gated-MLP middle: g, u (M, K) BF16 -> x = BF16(g * u) * su -> walsh -> per-token INT8 (q / q4, scale).
 * Replaces kernels.pre2 / k_pre2 (deploy/tcq_kernels/kernels.py:295-307, 631-633). */
int tcq_pre2(const void* g, const void* u, const int8_t* su, int8_t* q, int32_t* q4, int ldq, float* scale, int M, int K,
             tcq_stream_t stream);

/* ------------------------------------------------------------------------------------- norms around the projections */

/* Gemma RMSNorm of M rows of BF16 x (M, K) -> y (M, K) BF16: y = bf16((x * r) * (1 + w)), r = 1 / sqrt(sum(x^2) / K + eps) in
 * FP32, w (K,) BF16. The sum of squares runs in an order fixed by K alone (16-element chunk sums, then a pairwise tree), so
 * the fused kernels below reproduce this output bit for bit. K % 16 == 0. No reference counterpart: the reference leaves the
 * policy's norms to PyTorch (modules.py:226-243 only loads their weights); these kernels fuse them into the prologues. */
int tcq_rmsnorm(const void* x, const void* w, float eps, void* y, int M, int K, tcq_stream_t stream);

/* tcq_rmsnorm followed by tcq_pre with signs su, in one launch: q / q4 / scale of fwht(RMSNorm(x) * su). Extends the
 * rotate + quantize prologue kernels.pre (deploy/tcq_kernels/kernels.py:208-219) with the decoder layer's input norm. */
int tcq_norm_pre(const void* x, const void* w, float eps, const int8_t* su, int8_t* q, int32_t* q4, int ldq, float* scale, int M,
                 int K, tcq_stream_t stream);

/* Epilogue + residual + next prologue of a decoder layer, one launch: a = the tcq_post output of columns col0 .. col0 + N
 * (BF16 rounding), xout = bf16(x + a) (x, xout (M, N) BF16); then, when w is given, q / q4 / scale of
 * fwht(RMSNorm(xout) * su) as tcq_norm_pre. Extends kernels.post (deploy/tcq_kernels/kernels.py:221-230) with the residual
 * add and the following norm. N % 16 == 0. acc_dtype TCQ_I32 may carry TCQ_K_PARTS2 / TCQ_K_PARTS4 (power-of-two N of
 * 1024 .. 16384, 16-byte aligned operands; else TCQ_ERR_UNSUPPORTED). */
int tcq_post_add_norm_pre(const void* acc, int acc_dtype, int lda, int col0, const float* s, const float* rs, const int8_t* sv,
                          const float* bias, const void* x, void* xout, const void* w, float eps, const int8_t* su, int8_t* q,
                          int32_t* q4, int ldq, float* scale, int M, int N, tcq_stream_t stream);

/* Attention of H <= 8 query heads over one shared key / value head of dim D = 256 (multi-query), BF16 in and out, FP32
 * arithmetic. q (M, H * D); keys / values = the P cache rows (k_cache, v_cache (P, D); NULL when P = 0) followed by this
 * call's M rows (k_new, v_new (M, D)); query t sees key j iff causal_offset < 0 or j <= causal_offset + t. Scores
 * (q . k) / 16, softmax over the visible keys, computed in chunks of 64 keys (chunk maximum, exponentials, sums) merged
 * per token: the result depends on the number of keys only through that fixed chunking. part: workspace of
 * M * tcq_attend_chunks(P, M) * H * (D + 4) floats, 16-byte aligned. Outputs: o (M, H * D) BF16 (may be NULL when su is given) and, when su
 * is given, the rotate + quantize prologue of the next projection applied to the BF16 o row (q8 (M, H * D) int8, scale (M,)).
 * No reference counterpart: the reference policy's attention is PyTorch; this is the decoder layers' attention between
 * the TCQ projections, with the o-projection prologue (kernels.pre, deploy/tcq_kernels/kernels.py:208-219) fused in. */
int tcq_attend_chunks(int P, int M);
/* The first half of tcq_attend_q4: the chunk partials part ((M, tcq_attend_chunks(P, M), H, 260) FP32: o[256], m, l per
 * token, chunk and head) without the merge, for a product that merges them in its prologue (tcq_prologue.part). No
 * reference counterpart (the reference leaves attention to PyTorch). */
int tcq_attend_parts(const void* q, const void* k_cache, const void* v_cache, int P, const void* k_new, const void* v_new, int M,
                     int H, int D, int causal_offset, float* part, tcq_stream_t stream);
/* tcq_post_group of a one-token q / k / v product with FP32 z (acc_dtype TCQ_F32, no bias, output rotations on) followed
 * by tcq_attend_parts, in one launch: z_q (2048 = 8 heads x 256), z_k, z_v (256 each) the product's FP32 row segments
 * (16-byte aligned), sv_q / sv_k / sv_v their signs (8-byte aligned); q_t = bf16((walsh(z_t) * c_t) * sv_t), c_t =
 * 1 / sqrt(n_t), exactly as tcq_post_group. The new key and value rows are written to k_out / v_out (256 BF16 each, e.g.
 * row P of a preallocated cache) and take part as key P; the query row exists only inside the launch. part as
 * tcq_attend_parts with M = 1, H = 8, D = 256. No reference counterpart: it fuses the q / k / v epilogue
 * (kernels.postg, deploy/tcq_kernels/kernels.py:249-261) into this library's attention. */
int tcq_attend_post_parts(const float* z_q, const float* z_k, const float* z_v, const int8_t* sv_q, const int8_t* sv_k,
                          const int8_t* sv_v, const void* k_cache, const void* v_cache, int P, void* k_out, void* v_out, int H, int D,
                          int causal_offset, float* part, tcq_stream_t stream);
int tcq_attend(const void* q, const void* k_cache, const void* v_cache, int P, const void* k_new, const void* v_new, int M, int H,
               int D, int causal_offset, float* part, void* o, const int8_t* su, int8_t* q8, float* scale, tcq_stream_t stream);
/* tcq_attend whose prologue also writes the q4 output of the quantizing entry points (q4, ldq as tcq_pre; q8 may then be
 * NULL), e.g. the token-block layout the small-M product of the output projection reads. No reference counterpart. */
int tcq_attend_q4(const void* q, const void* k_cache, const void* v_cache, int P, const void* k_new, const void* v_new, int M, int H,
                  int D, int causal_offset, float* part, void* o, const int8_t* su, int8_t* q8, int32_t* q4, int ldq, float* scale,
                  tcq_stream_t stream);
/* tcq_attend_q4 without the workspace argument, for callers that cannot allocate device memory (code under HIP-graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. The workspace is a
 * file-scope device array of tcq_attend_static_floats() floats (8 MiB) on each device the library runs on, held until the
 * process ends; a call that needs more (M * tcq_attend_chunks(P, M) * H * 260 floats) returns TCQ_ERR_UNSUPPORTED before
 * launching. The call allocates nothing. Calls that overlap on one device share the array and race: order them (one stream,
 * or events between streams). */
int tcq_attend_q4_static(const void* q, const void* k_cache, const void* v_cache, int P, const void* k_new, const void* v_new, int M,
                         int H, int D, int causal_offset, void* o, const int8_t* su, int8_t* q8, int32_t* q4, int ldq, float* scale,
                         tcq_stream_t stream);
size_t tcq_attend_static_floats(void);

/* -------------------------------------------------------------------------------------------------------- products */

/* One layer of a batched FP16-table decode-GEMV / small-M GEMM (M <= 16 tokens): z[t, i] = (sum_k h16[t, k] *
 * Q[i, k]) * hscale[t] * row_scale[i], Q = FP16 table values decoded from wdev on the fly, FP32 accumulation (MFMA).
 * All layers of a batch share m, n, M, h16 and hscale. */
typedef struct tcq_gemv_layer {
    const void* wdev;       /* tcq_repack layout */
    const void* tlut;       /* (512, 2) FP16, or (G, 512, 2) row-group tables */
    const void* row_scale;  /* (m,) FP16 */
    float* z;               /* (M, m) FP32 out */
    int rows_per_table;     /* row-group tables: rows m / G per table (a multiple of 16); 0 = one table */
} tcq_gemv_layer;

/* layers: a DEVICE array of nlayers descriptors. The FP16-table product of tcq_format.reference_linear(table='fp16',
 * a8=False) (tcq_format.py:139-144), which the reference computes only in PyTorch (FP64 matmul); its INT8-table kernel
 * counterpart is kernels.gemmf_tcq / k_gemmf_tcq (kernels.py:465-489). */
int tcq_gemv_f16(const tcq_gemv_layer* layers, int nlayers, const void* h16, const float* hscale, int M, int m, int n,
                 tcq_stream_t stream);
/* The same for layers with row-group tables: every descriptor's rows_per_table must equal rows_per_table (the launch plan
 * keeps each workgroup inside one group). */
int tcq_gemv_f16_groups(const tcq_gemv_layer* layers, int nlayers, const void* h16, const float* hscale, int M, int m, int n,
                        int rows_per_table, tcq_stream_t stream);

/* One layer of a decode-GEMV stream with the output rotation fused: y (M, m) = walsh(z) * sv (+ bias) as tcq_post on the FP32
 * z of tcq_gemv_f16, stored as y_dtype (F16 / BF16 / F32). sv (m,) int8 and bias (m,) FP32 (or NULL) 16-byte aligned. */
typedef struct tcq_gemv_post_layer {
    const void* wdev;       /* tcq_repack layout */
    const void* tlut;       /* (512, 2) FP16 (one table) */
    const void* row_scale;  /* (m,) FP16 */
    int rows_per_table;     /* must be 0 */
    const int8_t* sv;       /* (m,) output signs */
    const float* bias;      /* (m,) FP32 or NULL */
    void* y;                /* (M, m) output */
} tcq_gemv_post_layer;

/* tcq_gemv_f16 + tcq_postg in one launch for layer streams: one workgroup per layer computes its whole z (M <= 16 rows of m
 * outputs kept in LDS) and rotates it, so z never goes to memory. Bit for bit the two launches when tcq_gemv_f16 runs its
 * layer-stream plan (from 256 layers on); its latency plan for small batches sums the K chunks in another order.
 * No reference counterpart (the reference's float path runs the product and the epilogue as separate kernels,
 * kernels.py:465-489, 612-615). */
int tcq_gemv_f16_post(const tcq_gemv_post_layer* layers, int nlayers, const void* h16, const float* hscale, int M, int m, int n,
                      int y_dtype, tcq_stream_t stream);

/* One whole layer in one launch, the FP16-table float path for a few tokens: y = walsh(walsh(x * su) Q^T * row_scale) * sv
 * (+ bias), i.e. tcq_pre_h16 + tcq_gemv_f16 (its latency plan) + tcq_post step for step, so y equals that three-launch chain
 * bit for bit. Replaces, for one layer, tcq_format.reference_linear(x, layer, a8=False, table='fp16')
 * (tcq_format.py:125-148, the float definition the reference's parity checks use).
 * x (M, n) F32 / BF16 / F16, M <= 16; wdev: tcq_repack words; tlut (512, 2) FP16; row_scale (m,) FP16; sv (m,); bias (m,)
 * FP32 or NULL; y (M, m) of y_dtype (F16 / BF16 / F32).
 * Workspace: z (M, m) FP32, 16-byte aligned (left holding walsh(x * su) Q^T * row_scale, the layer before its output
 * rotation; row_scale must be 8-byte aligned) and
 * *counter, one int that must be zero before the first call; every call leaves it zero, so the call can be captured in a
 * graph and replayed. Calls that share a workspace must not overlap. */
int tcq_layer_f16(const void* x, int x_dtype, const int8_t* su, const void* wdev, const void* tlut, const void* row_scale,
                  const int8_t* sv, const float* bias, void* y, int y_dtype, int M, int m, int n, float* z, int* counter,
                  tcq_stream_t stream);

/* The first two steps of that layer in one launch: z (M, m) FP32 = walsh(x * su) Q^T * row_scale, i.e. tcq_pre_h16 +
 * tcq_gemv_f16 (its latency plan) step for step, so z equals that two-launch chain bit for bit; tcq_post(z, ...) then gives
 * tcq_layer_f16's y. For one layer, the input rotation and the FP16-table product of tcq_format.reference_linear(table='fp16',
 * a8=False) (tcq_format.py:139-144); the reference's kernel counterparts are kernels.pre_h + kernels.gemmf_tcq
 * (kernels.py:309-317, 465-489). Arguments as tcq_layer_f16 (no workspace: z is the output). */
int tcq_pre_gemv_f16(const void* x, int x_dtype, const int8_t* su, const void* wdev, const void* tlut, const void* row_scale,
                     int M, int m, int n, float* z, tcq_stream_t stream);

/* One layer (segment) of a small-M INT8 product. The output of the segment starts at its first column: out[t * ldo + i] for
 * token t and output row i < m (the layers of a q/k/v or gate/up group write side by side into one (M, ldo) buffer). */
typedef struct tcq_gemm_seg {
    const void* w;       /* tcq_gemm_tcq: tcq_repack words of an (m, K) layer; tcq_gemm_w8: (m, K) int8 row-major weights */
    const int8_t* t8;    /* (512, 2) INT8 table, or (G, 512, 2) row-group tables (tcq_gemm_tcq only) */
    const float* rs;     /* (m,) FP32 row scale (unused for I32 output) */
    void* out;           /* output, first column of the segment */
    int m;               /* output rows, a multiple of 16 */
    int rows_per_table;  /* row-group tables: rows m / G per table (a multiple of 16); 0 = one table */
} tcq_gemm_seg;

/* W2A8 fused decode + product for M <= 64 tokens: acc[t, i] = sum_k q[t, k] * w8[i, k], exact in int32, with w8 = sign *
 * t8[hash(state)] decoded from the words on the fly. out_dtype F32: z = (float(acc) * s[t]) * rs[i]; BF16: its rounding;
 * I32: acc (with TCQ_K_PARTS2 / TCQ_K_PARTS4: its K parts, M <= 64). q (M, K) int8 row-major (or in the token-block
 * layout when out_dtype carries TCQ_Q_TOKEN_BLOCKS), s (M,) FP32, K a multiple of 16. segs: HOST array of nseg <= TCQ_MAX_SEGS descriptors
 * (copied into the launch). Replaces kernels.gemm_tcq / k_gemm_tcq (deploy/tcq_kernels/kernels.py:403-427, 671-673),
 * which takes at most three concatenated layers (q/k/v or gate/up, table chosen by tile-row bounds) and MT <= 10 tokens. */
int tcq_gemm_tcq(const tcq_gemm_seg* segs, int nseg, const int8_t* q, const float* s, int M, int K, int out_dtype, int ldo,
                 tcq_stream_t stream);

/* INT8-resident product, same contract with w = decoded (m, K) int8 weights (tcq_decode_i8). Replaces kernels.gemm_w8 /
 * k_gemm_w8 / k_gemm_w8d (deploy/tcq_kernels/kernels.py:365-399, 662-668). */
int tcq_gemm_w8(const tcq_gemm_seg* segs, int nseg, const int8_t* q, const float* s, int M, int K, int out_dtype, int ldo,
                tcq_stream_t stream);

/* Prologue of a one-token product, three forms. With acc: the arguments of tcq_post_add_norm_pre for M = 1 with the norm
 * (acc the previous product's int32 sums, acc_dtype TCQ_I32, optionally | TCQ_K_PARTS2 / TCQ_K_PARTS4 with part p at
 * acc + p * lda; s, rs, sv, bias its epilogue; x, xout the residual; w, eps the RMSNorm; su the signs of the product that
 * follows). Without acc, with part: the second half of tcq_attend_q4 for one token (the merge of the chunk partials part
 * of tcq_attend_parts, chunks = tcq_attend_chunks(P, 1), keys = P + 1, causal the causal offset or -1, heads = 8), then the
 * rotate + quantize of its BF16 row with signs su. Without acc and part: tcq_pre of the BF16 row x with signs su. Every
 * form may write copies of the INT8 row (q, K bytes) and its scale (scale: the token scale a later epilogue of int32 sums
 * needs). */
typedef struct {
    const void* acc;
    int acc_dtype;
    int lda, col0;
    const float* s;
    const float* rs;
    const int8_t* sv;
    const float* bias;
    const void* x;
    void* xout;
    const void* w;
    float eps;
    const int8_t* su;
    int8_t* q;
    float* scale;
    const float* part;   /* attention partials of tcq_attend_parts (acc NULL): the merge of their chunks is the prologue */
    int chunks, keys, causal, heads;
} tcq_prologue;

/* The prologue (tcq_post_add_norm_pre(pro..., M = 1, N = K), or tcq_pre(x, TCQ_BF16, su, ..., M = 1, K)) followed by
 * tcq_gemm_tcq / tcq_gemm_w8 of its INT8 row, in one launch: every workgroup computes the row itself (the same operations,
 * bit for bit) and multiplies it, so the row never leaves the chip and the chain loses a launch. Supported: with acc,
 * K = 2048, bias NULL, out_dtype TCQ_F32 (tcq_gemm_tcq: optionally | TCQ_Z_W128T); with part, K = 2048 (8 heads),
 * out_dtype TCQ_I32 (optionally | TCQ_K_PARTS2); with neither, K = 16384, out_dtype TCQ_I32 (optionally | TCQ_K_PARTS2);
 * else TCQ_ERR_UNSUPPORTED. 16-byte aligned operands. No reference counterpart: the
 * reference runs the epilogue, the residual add, the norm and the quantizer as separate steps (kernels.py:208-230; the
 * norm in PyTorch). */
int tcq_gemm_tcq_pro(const tcq_gemm_seg* segs, int nseg, const tcq_prologue* pro, int K, int out_dtype, int ldo, tcq_stream_t stream);
int tcq_gemm_w8_pro(const tcq_gemm_seg* segs, int nseg, const tcq_prologue* pro, int K, int out_dtype, int ldo, tcq_stream_t stream);

/* kernels.gemm_w8 / k_gemm_w8 (deploy/tcq_kernels/kernels.py:365-382, 662-668), argument for argument: W (N, K) int8 resident
 * weights, q4 (K/4, ldq) int32 activation words (the reference passes q4 (K/4, M), ldq = M), s (M,) FP32 token scales, rs (N,)
 * FP32 row scales, z (M, N) FP32 = (float(acc) * s[t]) * rs[i], acc exact in int32. M <= 64, N and K multiples of 16; z and
 * rs 16-byte aligned. */
int tcq_gemm_w8_q4(const int8_t* W, const int32_t* q4, int ldq, const float* s, const float* rs, float* z, int M, int N, int K,
                   tcq_stream_t stream);
/* kernels.gemm_tcq / k_gemm_tcq (deploy/tcq_kernels/kernels.py:403-427, 671-673), argument for argument: the fused decode +
 * product over the packed words as stored (bits (N/16 * K/16, 32) uint16, up to three layers concatenated along the rows,
 * no tcq_repack), t8 up to three concatenated (512, 2) INT8 tables, tile row I (16 output rows) decoded with table
 * (I >= nb0) + (I >= nb1) (the reference's bounds; 0 <= nb0 <= nb1); q4, s, rs, z as tcq_gemm_w8_q4. */
int tcq_gemm_tcq_q4(const void* bits, const int8_t* t8, const int32_t* q4, int ldq, const float* s, const float* rs, float* z, int M,
                    int N, int K, int nb0, int nb1, tcq_stream_t stream);

/* W8A8 INT8 GEMM: acc[m, n] = sum_k a[m, k] w[n, k], exact int32. a (M, K) int8 per-token quantized activations, w (N, K)
 * int8 per-output-channel quantized weights (both row-major, K a multiple of 16), out (M, ldo) of out_dtype: I32 the
 * accumulators; F32 (float(acc) * sa[m]) * sw[n]; BF16 the BF16 rounding of that (sa, sw FP32 scales, unused for I32).
 * Replaces the prefill product torch._int_mm(q, W.t()) of Group.product (deploy/tcq_kernels/modules.py:81-86;
 * tcq_format.int_matmul, tcq_format.py:110-116) followed by the (acc * s) * rs scaling of tcq_format.reference_linear
 * (tcq_format.py:135). Few tokens (M <= 16, or M <= 64 with N <= 8192) run the small-M product of tcq_gemm_w8 (one K chunk per wave), the
 * rest the tiled GEMM. */
int tcq_gemm_i8(const int8_t* a, const int8_t* w, const float* sa, const float* sw, void* out, int out_dtype, int ldo, int M, int N,
                int K, tcq_stream_t stream);

/* BF16 GEMM on dense BF16 weights: acc = sum_k a[m, k] w[n, k] with FP32 accumulation, a (M, K) BF16, w (N, K) BF16 (e.g.
 * the INT8 table values as BF16 from tcq_decode_f16 with the BF16 table); out = (acc * sa[m]) * sw[n] as FP32 or BF16
 * (sa / sw may be NULL: factor 1). K % 16 == 0, N % 4 == 0; a, w, out 16-byte aligned. Replaces the prefill product of the
 * reference's Group.run_float, `h @ W.t()` on BF16 weights decoded by kernels.decode_bf16 (deploy/tcq_kernels/modules.py:
 * 120-126), for callers that hold such dense weights; the module layer runs tcq_gemmf_* instead (no dense copy). */
int tcq_gemm_bf16(const void* a, const void* w, const float* sa, const float* sw, void* out, int out_dtype, int ldo, int M, int N,
                  int K, tcq_stream_t stream);

/* W2 float path prologue: bf16(fwht(x * su)) per token (x (M, K) of x_dtype F32 / BF16 / F16, contiguous) into h (M, K)
 * row-major and / or hT (K, ldh) with token = column (ldh >= M); either may be NULL, not both. Replaces kernels.pre_h /
 * k_preh_{bf16,f32} (deploy/tcq_kernels/kernels.py:309-317, 677-680), argument for argument. */
int tcq_pre_h(const void* x, int x_dtype, const int8_t* su, uint16_t* h, uint16_t* hT, int ldh, int M, int K, tcq_stream_t stream);

/* 1 when tcq_mid2 takes a gated-MLP middle of width N (N % 16 == 0, N <= 16384), else 0. Replaces kernels.mid2_available
 * (deploy/tcq_kernels/kernels.py:636-638), whose answer depends on the shared-memory limit of the reference's kernels. */
int tcq_mid2_available(int N);

/* The gated-MLP middle after a TCQ_Z_W128T product of gate | up (zt: gate's (M, 128, N / 128) block-transposed rows, then
 * up's), N = 16384, M <= 16: the remaining block Walsh stages (h = 128 .. N / 2), then as tcq_mid2 (* c, signs sv (2N,)
 * gate | up, BF16 roundings, GELU by the table, the product): p (M, N) BF16 = bf16(gelu(g) * u), natural order. tcq_pre
 * of p with the down projection's signs then gives tcq_mid2's q / q4 / scale bit for bit. Replaces, with the product's
 * epilogue, the one-workgroup tcq_mid2 of few tokens (kernels.py:263-278, 640-643) by work spread over many CUs. */
int tcq_glu_split(const float* zt, int N, const int8_t* sv, const uint16_t* gelu_lut, uint16_t* p, int M, tcq_stream_t stream);

/* W2 float path products over up to TCQ_MAX_SEGS layers side by side (segments as tcq_gemm_tcq): acc[t, i] = sum_k w[i, k]
 * h[t, k] with FP32 sums (MFMA blocks), the weights the INT8 table values taken as BF16, h (M, K) BF16 rotated activations
 * (tcq_pre_h / tcq_rht), any M (groups of 64 tokens over grid.z). out_dtype F32: out = acc * rs[i] (the expert's z,
 * kernels.py:430-439); BF16: out = bf16(acc), unscaled (the prefill product rounded to BF16, modules.py:126, scaled by rs
 * in tcq_post with a BF16 accumulator). ldo % 4 == 0, h 16-byte aligned, FP32 out / rs 16-byte aligned.
 * tcq_gemmf_tcq decodes the tcq_repack words of each segment on the fly (w = words, t8 its table or row-group tables);
 * tcq_gemmf_w8 reads resident INT8 weights (w = (m, K) int8, t8 unused). Replace kernels.gemmf_tcq / k_gemmf_tcq and
 * kernels.gemmf_w8 / k_gemmf_w8 (deploy/tcq_kernels/kernels.py:442-489, 689-696) in the module layer, and the prefill
 * product of Group.run_float (decode_bf16 + `h @ W.t()`, modules.py:120-126) without a dense BF16 copy. */
int tcq_gemmf_tcq(const tcq_gemm_seg* segs, int nseg, const void* h, int M, int K, int out_dtype, int ldo, tcq_stream_t stream);
int tcq_gemmf_w8(const tcq_gemm_seg* segs, int nseg, const void* h, int M, int K, int out_dtype, int ldo, tcq_stream_t stream);

/* kernels.gemmf_w8 / k_gemmf_w8 (deploy/tcq_kernels/kernels.py:442-463, 689-691), argument for argument: W (N, K) int8 resident
 * weights, hT (K, ldh) BF16 with token = column (the reference passes hT (K, M), ldh = M, from pre_h), rs (N,) FP32, z (M, N)
 * FP32 = acc * rs. N and K multiples of 16; z and rs 16-byte aligned; any M <= ldh. */
int tcq_gemmf_w8_hT(const int8_t* W, const void* hT, int ldh, const float* rs, float* z, int M, int N, int K, tcq_stream_t stream);
/* kernels.gemmf_tcq / k_gemmf_tcq (deploy/tcq_kernels/kernels.py:465-489, 694-696), argument for argument: the fused decode +
 * float product over the packed words as stored (bits (N/16 * K/16, 32) uint16, up to three layers concatenated along the
 * rows), t8 up to three concatenated (512, 2) INT8 tables, tile row I decoded with table (I >= nb0) + (I >= nb1); hT, rs, z
 * as tcq_gemmf_w8_hT. */
int tcq_gemmf_tcq_hT(const void* bits, const int8_t* t8, const void* hT, int ldh, const float* rs, float* z, int M, int N, int K,
                     int nb0, int nb1, tcq_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
