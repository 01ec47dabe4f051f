// Row kernels built on the LDS block-Walsh engine: randomized Hadamard (RHT), rotate + quantize, rotate for the float path,
// plain per-row quantizer, and the scale + rotate epilogue. One workgroup per token row; every butterfly is the FP32
// (a + b, a - b) of tcq_format.fwht in stage order h = 1, 2, 4, ... so the results equal the reference bit for bit.
#include "tcq_device.h"
#include "tcq_launch.h"

template <int DT> struct Elem;
template <> struct Elem<TCQ_F32> { static __device__ __forceinline__ float ld(const void* p, size_t i) { return ((const float*)p)[i]; }
                                  static __device__ __forceinline__ void st(void* p, size_t i, float v) { ((float*)p)[i] = v; } };
template <> struct Elem<TCQ_BF16> { static __device__ __forceinline__ float ld(const void* p, size_t i) { return bf16_to_f32(((const u16*)p)[i]); }
                                   static __device__ __forceinline__ void st(void* p, size_t i, float v) { ((u16*)p)[i] = f32_to_bf16(v); } };
template <> struct Elem<TCQ_F16> { static __device__ __forceinline__ float ld(const void* p, size_t i) { return f16_to_f32(((const u16*)p)[i]); }
                                  static __device__ __forceinline__ void st(void* p, size_t i, float v) { ((u16*)p)[i] = f32_to_f16(v); } };
template <> struct Elem<TCQ_I32> { static __device__ __forceinline__ float ld(const void* p, size_t i) { return (float)((const int*)p)[i]; }
                                  static __device__ __forceinline__ void st(void*, size_t, float) {} };

// x (rows at stride ldx) * su -> LDS row
template <int XDT>
__device__ __forceinline__ void load_signed_row(float* lds, const void* x, size_t base, const i8* su, int K) {
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
        float v = Elem<XDT>::ld(x, base + i);
        if (su) v = v * (float)su[i];
        lds[lds_slot(i)] = v;
    }
    __syncthreads();
}

// ------------------------------------------------------------------------------------------------------------------- RHT
template <int XDT, int YDT>
__global__ void k_rht(const void* x, int ldx, const i8* su, void* y, int ldy, int K) {
    extern __shared__ float lds[];
    const size_t tok = blockIdx.x;
    load_signed_row<XDT>(lds, x, tok * ldx, su, K);
    block_walsh(lds, K, [&](int i, float v) { Elem<YDT>::st(y, tok * ldy + i, v); });
}

// ------------------------------------------------------------------------------------------------------ rotate + quantize
template <int XDT>
__global__ void k_pre(const void* x, const i8* su, i8* q, int* q4, int ldq, float* scale, int K) {
    extern __shared__ float lds[];
    __shared__ float red[16];
    const int tok = blockIdx.x;
    load_signed_row<XDT>(lds, x, (size_t)tok * K, su, K);
    float mx = 0.f;
    block_walsh(lds, K, [&](int i, float v) { lds[lds_slot(i)] = v; mx = fmaxf(mx, fabsf(v)); });
    const float s = token_scale(block_max(mx, red));
    if (threadIdx.x == 0) scale[tok] = s;
    quantize_row(lds, s, q ? q + (size_t)tok * K : nullptr, q4, tok, K, ldq);
}

// -------------------------------------------------------------------------------------------- rotate for the float path
template <int XDT>
__global__ void k_pre_h16(const void* x, const i8* su, u16* h16, float* hscale, int K) {
    extern __shared__ float lds[];
    __shared__ float red[16];
    const int tok = blockIdx.x;
    load_signed_row<XDT>(lds, x, (size_t)tok * K, su, K);
    float mx = 0.f;
    block_walsh(lds, K, [&](int i, float v) { lds[lds_slot(i)] = v; mx = fmaxf(mx, fabsf(v)); });
    const float amax = block_max(mx, red);
    int e = 0;
    if (amax > 0.f && amax < __builtin_inff()) {
        frexpf(amax, &e);            // amax = f 2^e, f in [0.5, 1): floor(log2 amax) = e - 1
        e -= 15;                     // amax / 2^e in [2^14, 2^15)
    }
    if (threadIdx.x == 0) hscale[tok] = ldexpf(1.f, e);
    u16* out = h16 + (size_t)tok * K;
    for (int i = threadIdx.x; i < K; i += blockDim.x) out[i] = f32_to_f16(ldexpf(lds[lds_slot(i)], -e));
}

// ------------------------------------------------------------------------------------------------- per-row INT8 (no RHT)
template <int XDT>
__global__ void k_quantize_rows(const void* x, int ldx, i8* q, float* scale, int K) {
    extern __shared__ float lds[];
    __shared__ float red[16];
    const int row = blockIdx.x;
    float mx = 0.f;
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
        const float v = Elem<XDT>::ld(x, (size_t)row * ldx + i);
        lds[lds_slot(i)] = v;
        mx = fmaxf(mx, fabsf(v));
    }
    const float s = token_scale(block_max(mx, red));
    if (threadIdx.x == 0) scale[row] = s;
    quantize_row(lds, s, q + (size_t)row * K, nullptr, row, K, 0);
}

// ------------------------------------------------------------------------------------------------- scale + rotate epilogue
template <int ADT>
__device__ __forceinline__ float scaled_acc(const void* acc, size_t idx, float s, const float* rs, int i) {
    if (ADT == TCQ_I32) return ((float)((const int*)acc)[idx] * s) * rs[i];
    if (ADT == TCQ_BF16) return bf16_to_f32(((const u16*)acc)[idx]) * rs[i];
    return ((const float*)acc)[idx];
}

template <int ADT, int YDT>
__global__ void k_post(const void* acc, int lda, int col0, const float* s, const float* rs, const i8* sv, const float* bias,
                       void* y, int N) {
    extern __shared__ float lds[];
    const int tok = blockIdx.x;
    const size_t base = (size_t)tok * lda + col0;
    const float st = (ADT == TCQ_I32) ? s[tok] : 1.f;
    for (int i = threadIdx.x; i < N; i += blockDim.x) lds[lds_slot(i)] = scaled_acc<ADT>(acc, base + i, st, rs, i);
    __syncthreads();
    const size_t yb = (size_t)tok * N;
    block_walsh(lds, N, [&](int i, float v) {
        v = v * (float)sv[i];
        if (bias) v = v + bias[i];
        Elem<YDT>::st(y, yb + i, v);
    });
}

// Batched epilogue: workgroup (token, segment). Segments with N outside (0, maxN] are skipped (LDS is sized for maxN).
template <int ADT, int YDT>
__global__ void k_postg(const tcq_post_seg* segs, const float* s, const u16* gelu_lut, int maxN) {
    extern __shared__ float lds[];
    const tcq_post_seg S = segs[blockIdx.y];
    const int tok = blockIdx.x, N = S.N;
    if (N <= 0 || N > maxN) return;
    const size_t base = (size_t)tok * S.lda + S.col0;
    const float st = (ADT == TCQ_I32) ? s[tok] : 1.f;
    for (int i = threadIdx.x; i < N; i += blockDim.x) lds[lds_slot(i)] = scaled_acc<ADT>(S.acc, base + i, st, S.rs, i);
    __syncthreads();
    const size_t yb = (size_t)tok * N;
    const bool gl = YDT == TCQ_BF16 && S.gelu && gelu_lut;
    block_walsh(lds, N, [&](int i, float v) {
        v = v * (float)S.sv[i];
        if (S.bias) v = v + S.bias[i];
        if (gl) ((u16*)S.y)[yb + i] = gelu_lut[f32_to_bf16(v)];
        else Elem<YDT>::st(S.y, yb + i, v);
    });
}

// =========================================================================================================== C ABI
static int row_threads(int K) {
    const int top = 1 << (31 - __builtin_clz(K));
    int t = 64;
    while (t < 512 && t * 32 < top) t <<= 1;
    return t;
}
static size_t row_lds(int K) { return (size_t)lds_words(K) * sizeof(float); }

#define DISPATCH_X(dt, KERNEL, ...)                                                             \
    switch (dt) {                                                                               \
        case TCQ_F32: { KERNEL(TCQ_F32, __VA_ARGS__); break; }                                  \
        case TCQ_BF16: { KERNEL(TCQ_BF16, __VA_ARGS__); break; }                                \
        case TCQ_F16: { KERNEL(TCQ_F16, __VA_ARGS__); break; }                                  \
        default: return TCQ_ERR_DTYPE;                                                          \
    }

extern "C" int tcq_rht(const void* x, int x_dtype, int ldx, const int8_t* su, void* y, int y_dtype, int ldy, int M, int n,
                       tcq_stream_t stream) {
    if (!x || !y || M <= 0 || n <= 0 || ldx < n || ldy < n) return TCQ_ERR_ARG;
    if (n > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    const dim3 grid(M), block(row_threads(n));
    const size_t sh = row_lds(n);
    hipStream_t st = (hipStream_t)stream;
#define RHT_Y(XD, YD) launch_k(k_rht<XD, YD>, grid, block, sh, st, x, ldx, (const i8*)su, y, ldy, n)
#define RHT_X(XD, _)                                          \
    switch (y_dtype) {                                        \
        case TCQ_F32: RHT_Y(XD, TCQ_F32); break;              \
        case TCQ_BF16: RHT_Y(XD, TCQ_BF16); break;            \
        case TCQ_F16: RHT_Y(XD, TCQ_F16); break;              \
        default: return TCQ_ERR_DTYPE;                        \
    }
    DISPATCH_X(x_dtype, RHT_X, 0)
    return launch_status();
}

extern "C" int tcq_pre(const void* x, int x_dtype, const int8_t* su, int8_t* q, int32_t* q4, int ldq, float* scale, int M, int K,
                       tcq_stream_t stream) {
    if (!x || !scale || (!q && !q4) || M <= 0 || K <= 0 || (q4 && ldq < M)) return TCQ_ERR_ARG;
    if (K % 4 || K > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    const dim3 grid(M), block(row_threads(K));
    const size_t sh = row_lds(K);
    hipStream_t st = (hipStream_t)stream;
#define PRE(XD, _) launch_k(k_pre<XD>, grid, block, sh, st, x, (const i8*)su, (i8*)q, (int*)q4, ldq, scale, K)
    DISPATCH_X(x_dtype, PRE, 0)
    return launch_status();
}

extern "C" int tcq_pre_h16(const void* x, int x_dtype, const int8_t* su, void* h16, float* hscale, int M, int K,
                           tcq_stream_t stream) {
    if (!x || !h16 || !hscale || M <= 0 || K <= 0) return TCQ_ERR_ARG;
    if (K > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    const dim3 grid(M), block(row_threads(K));
    const size_t sh = row_lds(K);
    hipStream_t st = (hipStream_t)stream;
#define PREH(XD, _) launch_k(k_pre_h16<XD>, grid, block, sh, st, x, (const i8*)su, (u16*)h16, hscale, K)
    DISPATCH_X(x_dtype, PREH, 0)
    return launch_status();
}

extern "C" int tcq_quantize_rows(const void* x, int x_dtype, int ldx, int8_t* q, float* scale, int M, int K, tcq_stream_t stream) {
    if (!x || !q || !scale || M <= 0 || K <= 0 || ldx < K) return TCQ_ERR_ARG;
    if (K % 4 || K > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    const dim3 grid(M), block(row_threads(K));
    const size_t sh = row_lds(K);
    hipStream_t st = (hipStream_t)stream;
#define QROWS(XD, _) launch_k(k_quantize_rows<XD>, grid, block, sh, st, x, ldx, (i8*)q, scale, K)
    DISPATCH_X(x_dtype, QROWS, 0)
    return launch_status();
}

extern "C" int tcq_post(const void* acc, int acc_dtype, int lda, int col0, const float* s, const float* rs, const int8_t* sv,
                        const float* bias, void* y, int y_dtype, int M, int N, tcq_stream_t stream) {
    if (!acc || !sv || !y || M <= 0 || N <= 0 || col0 < 0 || lda < col0 + N) return TCQ_ERR_ARG;
    if ((acc_dtype == TCQ_I32 && (!s || !rs)) || (acc_dtype == TCQ_BF16 && !rs)) return TCQ_ERR_ARG;
    if (N > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    const dim3 grid(M), block(row_threads(N));
    const size_t sh = row_lds(N);
    hipStream_t st = (hipStream_t)stream;
#define POST_Y(AD, YD) launch_k(k_post<AD, YD>, grid, block, sh, st, acc, lda, col0, s, rs, (const i8*)sv, bias, y, N)
#define POST_A(AD)                                           \
    switch (y_dtype) {                                       \
        case TCQ_F32: POST_Y(AD, TCQ_F32); break;            \
        case TCQ_BF16: POST_Y(AD, TCQ_BF16); break;          \
        case TCQ_F16: POST_Y(AD, TCQ_F16); break;            \
        default: return TCQ_ERR_DTYPE;                       \
    }
    switch (acc_dtype) {
        case TCQ_I32: POST_A(TCQ_I32); break;
        case TCQ_F32: POST_A(TCQ_F32); break;
        case TCQ_BF16: POST_A(TCQ_BF16); break;
        default: return TCQ_ERR_DTYPE;
    }
    return launch_status();
}

extern "C" int tcq_postg(const tcq_post_seg* segs, int nseg, int acc_dtype, const float* s, const uint16_t* gelu_lut, int y_dtype,
                         int M, int maxN, tcq_stream_t stream) {
    if (!segs || nseg <= 0 || M <= 0 || maxN <= 0) return TCQ_ERR_ARG;
    if (acc_dtype == TCQ_I32 && !s) return TCQ_ERR_ARG;
    if (maxN > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    if (nseg > 65535) return TCQ_ERR_UNSUPPORTED;
    const dim3 grid(M, nseg), block(row_threads(maxN));
    const size_t sh = row_lds(maxN);
    hipStream_t st = (hipStream_t)stream;
#define POSTG_Y(AD, YD) launch_k(k_postg<AD, YD>, grid, block, sh, st, segs, s, (const u16*)gelu_lut, maxN)
#define POSTG_A(AD)                                          \
    switch (y_dtype) {                                       \
        case TCQ_F32: POSTG_Y(AD, TCQ_F32); break;           \
        case TCQ_BF16: POSTG_Y(AD, TCQ_BF16); break;         \
        case TCQ_F16: POSTG_Y(AD, TCQ_F16); break;           \
        default: return TCQ_ERR_DTYPE;                       \
    }
    switch (acc_dtype) {
        case TCQ_I32: POSTG_A(TCQ_I32); break;
        case TCQ_F32: POSTG_A(TCQ_F32); break;
        case TCQ_BF16: POSTG_A(TCQ_BF16); break;
        default: return TCQ_ERR_DTYPE;
    }
    return launch_status();
}
