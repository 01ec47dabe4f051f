// Row kernels built on the LDS block-Walsh engine: randomized Hadamard (RHT), rotate + quantize, rotate for the float path,
// plain per-row quantizer, and the scale + rotate epilogues. One workgroup per (token row[, segment]); every butterfly is
// the FP32 (a + b, a - b) of tcq_format.fwht in stage order h = 1, 2, 4, ... so the results equal the reference bit for bit.
//
// A row moves HBM -> LDS -> HBM in 16-byte vectors (8 elements per thread-step) whenever the row length is a multiple of 8
// and the rows are 16-byte aligned, else element by element; the Walsh passes run in LDS between the two.
#include "tcq_device.h"
#include "tcq_launch.h"
#include "tcq_rows.h"

namespace {

// ---------------------------------------------------------------------------------------------------- element access
template <int DT> struct Elem;
template <> struct Elem<TCQ_F32> {
    static __device__ __forceinline__ float ld(const void* p, size_t i) { return gptr((const float*)p)[i]; }
    static __device__ __forceinline__ void st(void* p, size_t i, float v) { gptr((float*)p)[i] = v; }
    static __device__ __forceinline__ void ld8(const void* p, size_t i, float (&v)[8]) {
        const uint4_t a = gptr((const uint4_t*)((const float*)p + i))[0], b = gptr((const uint4_t*)((const float*)p + i))[1];
#pragma unroll
        for (int k = 0; k < 4; ++k) { v[k] = __uint_as_float(a[k]); v[4 + k] = __uint_as_float(b[k]); }
    }
    static __device__ __forceinline__ void st8(void* p, size_t i, const float (&v)[8]) {
        uint4_t a, b;
#pragma unroll
        for (int k = 0; k < 4; ++k) { a[k] = __float_as_uint(v[k]); b[k] = __float_as_uint(v[4 + k]); }
        gptr((uint4_t*)((float*)p + i))[0] = a;
        gptr((uint4_t*)((float*)p + i))[1] = b;
    }
};
template <int DT> struct Elem16 {
    static __device__ __forceinline__ float cv(u16 h) { return DT == TCQ_BF16 ? bf16_to_f32(h) : f16_to_f32(h); }
    static __device__ __forceinline__ u16 cv(float f) { return DT == TCQ_BF16 ? f32_to_bf16(f) : f32_to_f16(f); }
    static __device__ __forceinline__ float ld(const void* p, size_t i) { return cv(gptr((const u16*)p)[i]); }
    static __device__ __forceinline__ void st(void* p, size_t i, float v) { gptr((u16*)p)[i] = cv(v); }
    static __device__ __forceinline__ void ld8(const void* p, size_t i, float (&v)[8]) {
        const uint4_t a = gptr((const uint4_t*)((const u16*)p + i))[0];
#pragma unroll
        for (int k = 0; k < 4; ++k) { v[2 * k] = cv((u16)(a[k] & 0xffffu)); v[2 * k + 1] = cv((u16)(a[k] >> 16)); }
    }
    static __device__ __forceinline__ void st8(void* p, size_t i, const float (&v)[8]) {
        u32 a[4];
        if constexpr (DT == TCQ_BF16) {
            bf16_pack<4>(v, a);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) a[k] = (u32)cv(v[2 * k]) | ((u32)cv(v[2 * k + 1]) << 16);
        }
        gptr((uint4_t*)((u16*)p + i))[0] = uint4_t{a[0], a[1], a[2], a[3]};
    }
};
template <> struct Elem<TCQ_BF16> : Elem16<TCQ_BF16> {};
template <> struct Elem<TCQ_F16> : Elem16<TCQ_F16> {};
template <> struct Elem<TCQ_I32> {
    static __device__ __forceinline__ float ld(const void* p, size_t i) { return (float)gptr((const int*)p)[i]; }
    static __device__ __forceinline__ void ld8i(const void* p, size_t i, int (&v)[8]) {
        const int4_t a = gptr((const int4_t*)((const int*)p + i))[0], b = gptr((const int4_t*)((const int*)p + i))[1];
#pragma unroll
        for (int k = 0; k < 4; ++k) { v[k] = a[k]; v[4 + k] = b[k]; }
    }
};

__device__ __forceinline__ void ld8_i8(const i8* p, int i, float (&v)[8]) {
    const u64 w = *gptr((const u64*)(p + i));
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = (float)(i8)(w >> (8 * k));
}
__device__ __forceinline__ void ld8_f32(const float* p, int i, float (&v)[8]) { Elem<TCQ_F32>::ld8(p, i, v); }

// ------------------------------------------------------------------------------------------------------ row movement
// x[base + i] (* su[i]) -> LDS slot of i, for i < K. vec: 8-element vectors (K % 8 == 0, x + base and su 16 / 8-byte aligned).
template <int XDT>
__device__ __forceinline__ void load_row(float* lds, const void* x, size_t base, const i8* su, int K, bool vec) {
    if (vec) {
        for (int i = 8 * threadIdx.x; i < K; i += 8 * blockDim.x) {
            float v[8], s[8];
            Elem<XDT>::ld8(x, base + i, v);
            if (su) {
                ld8_i8(su, i, s);
#pragma unroll
                for (int k = 0; k < 8; ++k) v[k] = v[k] * s[k];
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) lds[lds_slot(i + k)] = v[k];
        }
    } else {
        for (int i = threadIdx.x; i < K; i += blockDim.x) {
            float v = Elem<XDT>::ld(x, base + i);
            if (su) v = v * (float)gptr(su)[i];
            lds[lds_slot(i)] = v;
        }
    }
    __syncthreads();
}

// LDS row -> y[base + i] = f(i, v) for i < K (vec: as load_row). f8(i, v[8]) transforms 8 consecutive values in place.
template <int YDT, class F8, class F1>
__device__ __forceinline__ void store_row(const float* lds, void* y, size_t base, int K, bool vec, F8&& f8, F1&& f1) {
    if (vec) {
        for (int i = 8 * threadIdx.x; i < K; i += 8 * blockDim.x) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = lds[lds_slot(i + k)];
            f8(i, v);
            Elem<YDT>::st8(y, base + i, v);
        }
    } else {
        for (int i = threadIdx.x; i < K; i += blockDim.x) Elem<YDT>::st(y, base + i, f1(i, lds[lds_slot(i)]));
    }
}

// In-place normalised block Walsh of the LDS row (values stay in LDS); ends with a barrier.
__device__ __forceinline__ void walsh_inplace(float* lds, int K) {
    block_walsh(lds, K, [&](int i, float v) { lds[lds_slot(i)] = v; });
    __syncthreads();
}

__device__ __forceinline__ bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// ------------------------------------------------------------------------------------------------------------------- RHT
template <int XDT, int YDT>
__global__ void k_rht(const void* x, int ldx, const i8* su, void* y, int ldy, int K, int vec) {
    extern __shared__ float lds[];
    const size_t tok = blockIdx.x;
    load_row<XDT>(lds, x, tok * ldx, su, K, vec);
    walsh_inplace(lds, K);
    store_row<YDT>(lds, y, tok * ldy, K, vec, [](int, float(&)[8]) {}, [](int, float v) { return v; });
}

// W2 float path prologue with the transposed output: bf16(fwht(x * su)) of token `tok` into column tok of hT (K, ldh) and,
// when h is given, into row tok of h (M, K) (the reference's k_preh, deploy/tcq_kernels/kernels.py:309-317). The hT stores
// of one row are ldh elements apart; a token's values stay in one workgroup.
template <int XDT>
__global__ void k_pre_hT(const void* x, const i8* su, u16* h, u16* hT, int K, int ldh, int vec) {
    extern __shared__ float lds[];
    const size_t tok = blockIdx.x;
    load_row<XDT>(lds, x, tok * K, su, K, vec);
    walsh_inplace(lds, K);
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
        const u16 b = f32_to_bf16(lds[lds_slot(i)]);
        gptr(hT)[(size_t)i * ldh + tok] = b;
        if (h) gptr(h)[tok * K + i] = b;
    }
}

// raw element bits <-> FP32 for FP32 / BF16 / FP16 rows (2-byte types in the low 16 bits)
template <int DT>
__device__ __forceinline__ float bits_to_f32(u32 b) {
    if constexpr (DT == TCQ_F32) return __uint_as_float(b);
    else return Elem16<DT>::cv((u16)b);
}
template <int DT>
__device__ __forceinline__ u32 f32_to_bits(float f) {
    if constexpr (DT == TCQ_F32) return __float_as_uint(f);
    else return (u32)Elem16<DT>::cv(f);
}

// k_rht on the register + transpose engine for rows of 2^L (2^LE values per thread, rows and signs 16-byte aligned): the
// row comes in and goes out as coalesced spans through LDS; x * su -> Walsh -> * c, the same operations as k_rht.
template <int XDT, int YDT, int L, int LE>
__global__ __launch_bounds__(1 << (L - LE)) void k_rht_tw(const void* x, int ldx, const i8* su, void* y, int ldy) {
    constexpr int E = 1 << LE, XS = XDT == TCQ_F32 ? 4 : 2, YS = YDT == TCQ_F32 ? 4 : 2;
    extern __shared__ float xs[];
    const size_t tok = blockIdx.x;
    const int i0 = E * threadIdx.x;
    Raw16<1> s0[E / 16];
    if (su) {
#pragma unroll
        for (int h = 0; h < E / 16; ++h) s0[h] = raw16<1>(su + i0 + 16 * h, true);
    }
    // the thread's 2^LE contiguous inputs (layout 0) straight from memory: each lane reads its own 16-byte pieces, which
    // costs the address unit more lines per instruction than lane-contiguous loads but saves the LDS round trip that would
    // bring lane-contiguous pieces into layout 0 (MI355X, BF16, 800 x 16384: 18.85 -> 15.87 us; FP32 20.7 -> 18.4 us)
    float v[E];
    {
        constexpr int NQ = E * XS / 16;
        const uint4_t* src = (const uint4_t*)((const char*)x + tok * ldx * XS + (size_t)i0 * XS);
        uint4_t raw[NQ];
#pragma unroll
        for (int j = 0; j < NQ; ++j) raw[j] = *gptr(src + j);
#pragma unroll
        for (int k = 0; k < E; ++k)
            v[k] = XS == 4 ? bits_to_f32<XDT>(raw[k >> 2][k & 3]) : bits_to_f32<XDT>((raw[k >> 3][(k & 7) >> 1] >> (16 * (k & 1))) & 0xffffu);
    }
    if (su) {
#pragma unroll
        for (int h = 0; h < E / 16; ++h) {
            float sg[16];
            cv16(s0[h], sg);
#pragma unroll
            for (int k = 0; k < 16; ++k) v[16 * h + k] = v[16 * h + k] * sg[k];
        }
    }
    tw_walsh<L, LE>(v, xs);
    const float c = (float)(1.0 / __builtin_sqrt((double)(1 << L)));
#pragma unroll
    for (int k = 0; k < E; ++k) v[k] = v[k] * c;
    tw_put<L, LE, 2>(v, xs);
    __syncthreads();
    tw_span_store<LE, YDT>((char*)y + tok * ldy * YS, xs);
}

// ------------------------------------------------------------------------------------------------------ rotate + quantize
// k_pre on the register + transpose engine for rows of 2^L without column scales (rows, signs and q 16-byte aligned): the
// thread's 2^LE contiguous inputs straight into registers as k_rht_tw loads them, * su, then tw_rotate_quantize (Walsh, * c,
// row max, INT8): the operations of k_pre in the same order.
template <int XDT, int L, int LE>
__global__ __launch_bounds__(1 << (L - LE)) void k_pre_tw(const void* x, const i8* su, i8* q, int* q4, int ldq, float* scale) {
    constexpr int E = 1 << LE, XS = XDT == TCQ_F32 ? 4 : 2, NQ = E * XS / 16;
    extern __shared__ float xs[];
    __shared__ float red[16];
    const int tok = blockIdx.x, i0 = E * threadIdx.x;
    Raw16<1> s0[E / 16];
    if (su) {
#pragma unroll
        for (int h = 0; h < E / 16; ++h) s0[h] = raw16<1>(su + i0 + 16 * h, true);
    }
    const uint4_t* src = (const uint4_t*)((const char*)x + ((size_t)tok << L) * XS + (size_t)i0 * XS);
    uint4_t raw[NQ];
#pragma unroll
    for (int j = 0; j < NQ; ++j) raw[j] = *gptr(src + j);
    float v[E];
#pragma unroll
    for (int k = 0; k < E; ++k)
        v[k] = XS == 4 ? bits_to_f32<XDT>(raw[k >> 2][k & 3]) : bits_to_f32<XDT>((raw[k >> 3][(k & 7) >> 1] >> (16 * (k & 1))) & 0xffffu);
    if (su) {
#pragma unroll
        for (int h = 0; h < E / 16; ++h) {
            float sg[16];
            cv16(s0[h], sg);
#pragma unroll
            for (int k = 0; k < 16; ++k) v[16 * h + k] = v[16 * h + k] * sg[k];
        }
    }
    tw_rotate_quantize<L, LE>(v, xs, red, q, q4, ldq, scale, tok);
}

// cs: FP16 column scales of the rotated activations (NULL: none), applied after the rotation, before the absmax.
template <int XDT>
__global__ void k_pre(const void* x, const i8* su, i8* q, int* q4, int ldq, float* scale, int K, int vec, const u16* cs) {
    extern __shared__ float lds[];
    __shared__ float red[16];
    const int tok = blockIdx.x;
    load_row<XDT>(lds, x, (size_t)tok * K, su, K, vec);
    float mx = 0.f;
    if (cs) {
        block_walsh(lds, K, [&](int i, float v) {
            const float w = v * f16_to_f32(gptr(cs)[i]);
            lds[lds_slot(i)] = w;
            mx = fmaxf(mx, fabsf(w));
        });
    } else {
        block_walsh(lds, K, [&](int i, float v) { lds[lds_slot(i)] = v; mx = fmaxf(mx, fabsf(v)); });
    }
    const float s = token_scale(block_max(mx, red));
    if (threadIdx.x == 0) scale[tok] = s;
    quantize_row(lds, s, q ? q + (size_t)tok * K : nullptr, q4, tok, K, ldq);
}

// -------------------------------------------------------------------------------------------- rotate for the float path
template <int XDT>
__global__ void k_pre_h16(const void* x, const i8* su, u16* h16, float* hscale, int K, int vec) {
    extern __shared__ float lds[];
    __shared__ float red[16];
    const int tok = blockIdx.x;
    load_row<XDT>(lds, x, (size_t)tok * K, su, K, vec);
    float mx = 0.f;
    block_walsh(lds, K, [&](int i, float v) { lds[lds_slot(i)] = v; mx = fmaxf(mx, fabsf(v)); });
    const float amax = block_max(mx, red);
    int e = 0;
    if (amax > 0.f && amax < __builtin_inff()) {
        frexpf(amax, &e);            // amax = f 2^e, f in [0.5, 1): floor(log2 amax) = e - 1
        e -= 15;                     // amax / 2^e in [2^14, 2^15)
    }
    if (threadIdx.x == 0) hscale[tok] = ldexpf(1.f, e);
    store_row<TCQ_F16>(lds, h16, (size_t)tok * K, K, vec, [&](int, float(&v)[8]) {
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = ldexpf(v[k], -e);
    }, [&](int, float v) { return ldexpf(v, -e); });
}

// k_pre_h16 for few rows of 2^L = 1024 / 2048 on the no-transpose engine (NWP = 2^L / 256 waves, 4 values per thread): the
// same sign products, butterflies, constant, maximum and scaling as k_pre_h16.
template <int XDT, int L, int NWP>
__global__ __launch_bounds__(64 * NWP) void k_pre_h16_wv(const void* x, const i8* su, u16* h16, float* hscale) {
    constexpr int K = 1 << L;
    __shared__ float xs[K];
    __shared__ float red[NWP];
    const int tok = blockIdx.x, t = threadIdx.x, lane = t & 63, w = t >> 6;
    const size_t i0 = (size_t)tok * K + 4 * t;
    float v[4];
    if constexpr (XDT == TCQ_F32) {
        const float4_t a = *gptr((const float4_t*)((const float*)x + i0));
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = a[k];
    } else {
        const uint2_t a = *gptr((const uint2_t*)((const u16*)x + i0));
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = Elem16<XDT>::cv((u16)(a[k >> 1] >> (16 * (k & 1))));
    }
    if (su) {
        const u32 sg = *gptr((const u32*)(su + 4 * t));
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = v[k] * (float)(i8)(sg >> (8 * k));
    }
    wave_walsh<2, NWP>(v, xs, [] { __syncthreads(); });
    const float c = (float)(1.0 / __builtin_sqrt((double)K));
    float mx = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        v[k] = v[k] * c;
        mx = fmaxf(mx, fabsf(v[k]));
    }
    mx = wave_max(mx);
    if (lane == 0) red[w] = mx;
    __syncthreads();
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < NWP; ++i) amax = fmaxf(amax, red[i]);
    int e = 0;
    if (amax > 0.f && amax < __builtin_inff()) {
        frexpf(amax, &e);
        e -= 15;
    }
    if (t == 0) hscale[tok] = ldexpf(1.f, e);
    *gptr((uint2_t*)(h16 + i0)) = uint2_t{(u32)f32_to_f16(ldexpf(v[0], -e)) | ((u32)f32_to_f16(ldexpf(v[1], -e)) << 16),
                                         (u32)f32_to_f16(ldexpf(v[2], -e)) | ((u32)f32_to_f16(ldexpf(v[3], -e)) << 16)};
}

// k_pre_h16 on the register engine for power-of-two rows of 256 .. 16384 (thread t < K / 16 owns elements [16 t, 16 t + 16),
// 16-byte loads and stores): the same sign products, butterflies, constant, maximum and scaling as k_pre_h16.
template <int XDT>
__global__ __launch_bounds__(1024) void k_pre_h16_reg(const void* x, const i8* su, u16* h16, float* hscale, int K) {
    extern __shared__ float xs[];                                      // K floats: the engine's exchange buffer
    __shared__ float red[16];
    const int tok = blockIdx.x, t = threadIdx.x;
    const bool on = t < (K >> 4);
    float v[16];
    if (on) {
        const size_t i0 = (size_t)tok * K + 16 * t;
        if constexpr (XDT == TCQ_F32) {
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const uint4_t a = gptr((const uint4_t*)((const float*)x + i0))[h];
#pragma unroll
                for (int k = 0; k < 4; ++k) v[4 * h + k] = __uint_as_float(a[k]);
            }
        } else {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint4_t a = gptr((const uint4_t*)((const u16*)x + i0))[h];
#pragma unroll
                for (int k = 0; k < 8; ++k) v[8 * h + k] = Elem16<XDT>::cv((u16)(a[k >> 1] >> (16 * (k & 1))));
            }
        }
        if (su) {
            float sg[16];
            cv16(raw16<1>(su + 16 * t, true), sg);
#pragma unroll
            for (int k = 0; k < 16; ++k) v[k] = v[k] * sg[k];
        }
    }
    reg_walsh16_part(v, K, xs);
    const float c = (float)(1.0 / __builtin_sqrt((double)K));
    float mx = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        v[k] = v[k] * c;
        if (on) mx = fmaxf(mx, fabsf(v[k]));
    }
    const float amax = block_max(mx, red);
    int e = 0;
    if (amax > 0.f && amax < __builtin_inff()) {
        frexpf(amax, &e);
        e -= 15;
    }
    if (t == 0) hscale[tok] = ldexpf(1.f, e);
    if (!on) return;
    uint4_t o[2];
#pragma unroll
    for (int k = 0; k < 8; ++k)
        o[k >> 2][k & 3] = (u32)f32_to_f16(ldexpf(v[2 * k], -e)) | ((u32)f32_to_f16(ldexpf(v[2 * k + 1], -e)) << 16);
    uint4_t* out = (uint4_t*)(h16 + (size_t)tok * K + 16 * t);
    gptr(out)[0] = o[0];
    gptr(out)[1] = o[1];
}

// ------------------------------------------------------------------------------------------------- per-row INT8 (no RHT)
template <int XDT>
__global__ void k_quantize_rows(const void* x, int ldx, i8* q, float* scale, int K, int vec) {
    extern __shared__ float lds[];
    __shared__ float red[16];
    const int row = blockIdx.x;
    load_row<XDT>(lds, x, (size_t)row * ldx, nullptr, K, vec);
    float mx = 0.f;
    for (int i = threadIdx.x; i < K; i += blockDim.x) mx = fmaxf(mx, fabsf(lds[lds_slot(i)]));
    const float s = token_scale(block_max(mx, red));
    if (threadIdx.x == 0) scale[row] = s;
    quantize_row(lds, s, q + (size_t)row * K, nullptr, row, K, 0);
}

// ------------------------------------------------------------------------------------------------- scale + rotate epilogue
// Accumulator column i of a row -> FP32: I32 (float(a) * s) * rs[i]; BF16 bf16(a) * rs[i]; F32 a (already scaled).
// This thread's first 8-element vector of an accumulator row (raw words: 32 bytes of FP32 / INT32, 16 of BF16) and of its
// row scales, loaded ahead of the rest of the row (vec rows only).
struct AccVec {
    uint4_t a[2], r[2];
};
template <int ADT>
__device__ __forceinline__ void load_acc_vec(AccVec& p, const void* acc, size_t base, const float* rs, int i) {
    if (ADT == TCQ_BF16) {
        p.a[0] = gptr((const uint4_t*)((const u16*)acc + base + i))[0];
    } else {
        p.a[0] = gptr((const uint4_t*)((const u32*)acc + base + i))[0];
        p.a[1] = gptr((const uint4_t*)((const u32*)acc + base + i))[1];
    }
    if (ADT != TCQ_F32) {
        p.r[0] = gptr((const uint4_t*)(rs + i))[0];
        p.r[1] = gptr((const uint4_t*)(rs + i))[1];
    }
}

template <int ADT>
__device__ __forceinline__ void load_acc_row(float* lds, const void* acc, size_t base, float s, const float* rs, int N, bool vec,
                                             bool pre = false, const AccVec& p0 = AccVec{}) {
    if (vec) {
        for (int i = 8 * threadIdx.x; i < N; i += 8 * blockDim.x) {
            float v[8];
            if (pre && i == 8 * (int)threadIdx.x) {
                float r[8];
#pragma unroll
                for (int k = 0; k < 4; ++k) { r[k] = __uint_as_float(p0.r[0][k]); r[4 + k] = __uint_as_float(p0.r[1][k]); }
                if (ADT == TCQ_I32) {
#pragma unroll
                    for (int k = 0; k < 8; ++k) v[k] = ((float)(int)p0.a[k >> 2][k & 3] * s) * r[k];
                } else if (ADT == TCQ_BF16) {
#pragma unroll
                    for (int k = 0; k < 8; ++k) v[k] = bf16_to_f32((u16)(p0.a[0][k >> 1] >> (16 * (k & 1)))) * r[k];
                } else {
#pragma unroll
                    for (int k = 0; k < 8; ++k) v[k] = __uint_as_float(p0.a[k >> 2][k & 3]);
                }
            } else if (ADT == TCQ_I32) {
                int a[8];
                float r[8];
                Elem<TCQ_I32>::ld8i(acc, base + i, a);
                ld8_f32(rs, i, r);
#pragma unroll
                for (int k = 0; k < 8; ++k) v[k] = ((float)a[k] * s) * r[k];
            } else if (ADT == TCQ_BF16) {
                float r[8];
                Elem<TCQ_BF16>::ld8(acc, base + i, v);
                ld8_f32(rs, i, r);
#pragma unroll
                for (int k = 0; k < 8; ++k) v[k] = v[k] * r[k];
            } else {
                Elem<TCQ_F32>::ld8(acc, base + i, v);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) lds[lds_slot(i + k)] = v[k];
        }
    } else {
        for (int i = threadIdx.x; i < N; i += blockDim.x) {
            float v;
            if (ADT == TCQ_I32) v = (Elem<TCQ_I32>::ld(acc, base + i) * s) * gptr(rs)[i];
            else if (ADT == TCQ_BF16) v = Elem<TCQ_BF16>::ld(acc, base + i) * gptr(rs)[i];
            else v = Elem<TCQ_F32>::ld(acc, base + i);
            lds[lds_slot(i)] = v;
        }
    }
    __syncthreads();
}

// y = walsh(row) * sv (+ bias) [-> GELU table for BF16 outputs]
// (sv0, b0: the signs and bias of this thread's first 8-element vector, loaded ahead with the accumulator row; vec only)
struct PostSide {
    u64 sv;
    uint4_t b[2];
};
__device__ __forceinline__ void load_post_side(PostSide& p, const i8* sv, const float* bias, int i) {
    p.sv = *gptr((const u64*)(sv + i));
    if (bias) {
        p.b[0] = gptr((const uint4_t*)(bias + i))[0];
        p.b[1] = gptr((const uint4_t*)(bias + i))[1];
    }
}
template <int YDT>
__device__ __forceinline__ void store_post_row(const float* lds, void* y, size_t base, const i8* sv, const float* bias,
                                               const u16* gelu, int N, bool vec, bool pre = false,
                                               const PostSide& p0 = PostSide{}) {
    store_row<YDT>(lds, y, base, N, vec, [&](int i, float(&v)[8]) {
        const bool first = pre && i == 8 * (int)threadIdx.x;
        float s[8];
        if (first) {
#pragma unroll
            for (int k = 0; k < 8; ++k) s[k] = (float)(i8)(p0.sv >> (8 * k));
        } else {
            ld8_i8(sv, i, s);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = v[k] * s[k];
        if (bias) {
            float b[8];
            if (first) {
#pragma unroll
                for (int k = 0; k < 4; ++k) { b[k] = __uint_as_float(p0.b[0][k]); b[4 + k] = __uint_as_float(p0.b[1][k]); }
            } else {
                ld8_f32(bias, i, b);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = v[k] + b[k];
        }
        if (YDT == TCQ_BF16 && gelu) {
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = bf16_to_f32(gptr(gelu)[f32_to_bf16(v[k])]);
        }
    }, [&](int i, float v) {
        v = v * (float)gptr(sv)[i];
        if (bias) v = v + gptr(bias)[i];
        if (YDT == TCQ_BF16 && gelu) v = bf16_to_f32(gptr(gelu)[f32_to_bf16(v)]);
        return v;
    });
}

template <int ADT, int YDT>
__global__ void k_post(const void* acc, int lda, int col0, const float* s, const float* rs, const i8* sv, const float* bias,
                       void* y, int N, int vec) {
    extern __shared__ float lds[];
    const int tok = blockIdx.x;
    PostSide p0{};
    const bool has0 = vec && 8 * (int)threadIdx.x < N;
    if (has0) load_post_side(p0, sv, bias, 8 * threadIdx.x);
    load_acc_row<ADT>(lds, acc, (size_t)tok * lda + col0, ADT == TCQ_I32 ? s[tok] : 1.f, rs, N, vec);
    walsh_inplace(lds, N);
    store_post_row<YDT>(lds, y, (size_t)tok * N, sv, bias, nullptr, N, vec, has0, p0);
}

// Batched epilogue: workgroup (token, segment). Segments with N outside (0, maxN], or without the row scale their
// accumulator type needs, are skipped (the host wrappers reject them before they get here). SEGS is a device array of
// descriptors (tcq_postg) or a by-value pack of at most TCQ_MAX_SEGS (tcq_post_group), indexed the same way.
// Vectors are used for a segment when its N is a multiple of 8 and its pointers and strides are 16-byte aligned.
struct PostPack {
    tcq_post_seg s[TCQ_MAX_SEGS];
    __device__ __forceinline__ const tcq_post_seg& operator[](int i) const { return s[i]; }
};

template <int ADT, int YDT, class SEGS>
__global__ void k_postg(SEGS segs, const float* s, const u16* gelu_lut, int maxN) {
    extern __shared__ float lds[];
    const tcq_post_seg S = segs[blockIdx.y];
    const int tok = blockIdx.x, N = S.N;
    if (N <= 0 || N > maxN || (ADT != TCQ_F32 && !S.rs)) return;
    const int esz = ADT == TCQ_BF16 ? 2 : 4, ysz = YDT == TCQ_F32 ? 4 : 2;
    const bool vec = N % 8 == 0 && aligned16(S.acc) && ((size_t)S.lda * esz) % 16 == 0 && ((size_t)S.col0 * esz) % 16 == 0 &&
                     aligned16(S.y) && ((size_t)N * ysz) % 16 == 0 && ((uintptr_t)S.sv & 7) == 0 && (!S.rs || aligned16(S.rs)) &&
                     (!S.bias || aligned16(S.bias));
    PostSide p0{};
    const bool has0 = vec && 8 * (int)threadIdx.x < N;
    if (has0) load_post_side(p0, S.sv, S.bias, 8 * threadIdx.x);
    load_acc_row<ADT>(lds, S.acc, (size_t)tok * S.lda + S.col0, ADT == TCQ_I32 ? s[tok] : 1.f, S.rs, N, vec);
    walsh_inplace(lds, N);
    store_post_row<YDT>(lds, S.y, (size_t)tok * N, S.sv, S.bias, S.gelu ? gelu_lut : nullptr, N, vec, has0, p0);
}

// RMSNorm of the LDS row (BF16 values as FP32) given its sum of squares: v <- bf16((v * r) * (1 + w[i])) * su[i] (su may be
// NULL), r = 1 / sqrt(ss / K + eps). Ends with a barrier.
// pre: w0 / su0 hold this thread's first chunk of w / su, loaded ahead.
__device__ __forceinline__ void norm_apply(float* lds, float ss, const u16* w, const i8* su, float eps, int K, bool vec,
                                           bool pre = false, const Raw16<2>& w0 = Raw16<2>{}, const Raw16<1>& su0 = Raw16<1>{}) {
    const float r = 1.f / __builtin_sqrtf(ss / (float)K + eps);
    for (int j = threadIdx.x; j < (K >> 4); j += blockDim.x) {
        float wv[16], sg[16];
        const bool first = pre && j == (int)threadIdx.x;
        if (first) cv16(w0, wv);
        else c16_bf16(w + 16 * j, vec, wv);
        if (su) {
            if (first) cv16(su0, sg);
            else c16_i8(su + 16 * j, vec, sg);
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            float v = bf16_to_f32(f32_to_bf16((lds[lds_slot(16 * j + k)] * r) * (1.f + wv[k])));
            if (su) v = v * sg[k];
            lds[lds_slot(16 * j + k)] = v;
        }
    }
    __syncthreads();
}

// Rotate + quantize the LDS row (values already signed): walsh, per-token absmax, INT8 (as k_pre).
__device__ __forceinline__ void rotate_quantize(float* lds, float* red, i8* q, int* q4, int ldq, float* scale, int tok, int K) {
    float mx = 0.f;
    block_walsh(lds, K, [&](int i, float v) { lds[lds_slot(i)] = v; mx = fmaxf(mx, fabsf(v)); });
    const float sc = token_scale(block_max(mx, red));
    if (threadIdx.x == 0) scale[tok] = sc;
    quantize_row(lds, sc, q ? q + (size_t)tok * K : nullptr, q4, tok, K, ldq);
}

// ------------------------------------------------------------------------------------------------------------ MLP middles
// Rounding points of the fused MLP middles (each stage is the unfused chain's): GELU and the gate / up products round to
// BF16 exactly where the separate epilogue + prologue kernels would store BF16 tensors. GELU comes from the 65536-entry
// table (lut) of PyTorch's own results; its 16 lookups per chunk are issued together.
__device__ __forceinline__ void gelu16(const u16* lut, const float (&v)[16], u16 (&g)[16]) {
    u16 b[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) b[k] = f32_to_bf16(v[k]);
#pragma unroll
    for (int k = 0; k < 16; ++k) g[k] = gptr(lut)[b[k]];
}

// Gated MLP (down(gelu(gate(x)) * up(x))): accumulator row = gate columns [0, N) | up columns [N, 2N), scaled like tcq_post
// (rs and sv are the concatenated 2N vectors). g = GELU(BF16(walsh(gate) * sv)) is kept in LDS as BF16, then
// x = BF16(g * BF16(walsh(up) * sv)) * su -> walsh -> per-token INT8 of the down projection's input.
template <int ADT>
__global__ void k_mid2(const void* acc, int lda, const float* s, const float* rs, const i8* sv, const u16* lut, const i8* su,
                       i8* q, int* q4, int ldq, float* scale, int N, int vec, int svec) {
    extern __shared__ float lds[];
    __shared__ float red[16];
    u16* g = (u16*)(lds + lds_words(N));
    const int tok = blockIdx.x, j0 = threadIdx.x;
    const float st = ADT == TCQ_I32 ? s[tok] : 1.f;
    const bool has0 = j0 < (N >> 4);
    Raw16<1> svg0{}, svu0{}, sn0{};                                     // this thread's first chunk of sv (gate, up) and su
    if (has0) {
        svg0 = raw16<1>(sv + 16 * j0, svec);
        svu0 = raw16<1>(sv + N + 16 * j0, svec);
        sn0 = raw16<1>(su + 16 * j0, svec);
    }
    AccVec up0{};                                                       // first vector of the up half, loaded ahead
    const bool hasv = vec && 8 * (int)threadIdx.x < N;
    if (hasv) load_acc_vec<ADT>(up0, acc, (size_t)tok * lda + N, rs + (ADT == TCQ_F32 ? 0 : N), 8 * threadIdx.x);
    load_acc_row<ADT>(lds, acc, (size_t)tok * lda, st, rs, N, vec);
    walsh_inplace(lds, N);
    for (int j = j0; j < (N >> 4); j += blockDim.x) {
        float sg[16], v[16];
        u16 gv[16];
        if (j == j0) cv16(svg0, sg);
        else c16_i8(sv + 16 * j, svec, sg);
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = lds[lds_slot(16 * j + k)] * sg[k];
        gelu16(lut, v, gv);
#pragma unroll
        for (int k = 0; k < 16; ++k) g[16 * j + k] = gv[k];
    }
    __syncthreads();
    load_acc_row<ADT>(lds, acc, (size_t)tok * lda + N, st, rs + (ADT == TCQ_F32 ? 0 : N), N, vec, hasv, up0);
    walsh_inplace(lds, N);
    for (int j = j0; j < (N >> 4); j += blockDim.x) {
        float sg[16], sn[16];
        if (j == j0) {
            cv16(svu0, sg);
            cv16(sn0, sn);
        } else {
            c16_i8(sv + N + 16 * j, svec, sg);
            c16_i8(su + 16 * j, svec, sn);
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const float u = bf16_to_f32(f32_to_bf16(lds[lds_slot(16 * j + k)] * sg[k]));
            lds[lds_slot(16 * j + k)] = bf16_to_f32(f32_to_bf16(bf16_to_f32(g[16 * j + k]) * u)) * sn[k];
        }
    }
    __syncthreads();
    rotate_quantize(lds, red, q, q4, ldq, scale, tok, N);
}

// Plain MLP (fc2(gelu(fc1(x)))): x = GELU(BF16(walsh(acc) * sv + bias)) * su -> walsh -> per-token INT8 of fc2's input.
template <int ADT>
__global__ void k_mid1(const void* acc, int lda, const float* s, const float* rs, const i8* sv, const float* bias, const u16* lut,
                       const i8* su, i8* q, int* q4, int ldq, float* scale, int N, int vec, int svec) {
    extern __shared__ float lds[];
    __shared__ float red[16];
    const int tok = blockIdx.x;
    load_acc_row<ADT>(lds, acc, (size_t)tok * lda, ADT == TCQ_I32 ? s[tok] : 1.f, rs, N, vec);
    walsh_inplace(lds, N);
    for (int j = threadIdx.x; j < (N >> 4); j += blockDim.x) {
        float sg[16], sn[16], b[16], v[16];
        u16 gv[16];
        c16_i8(sv + 16 * j, svec, sg);
        c16_i8(su + 16 * j, svec, sn);
        if (bias) c16_f32(bias + 16 * j, svec, b);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            v[k] = lds[lds_slot(16 * j + k)] * sg[k];
            if (bias) v[k] = v[k] + b[k];
        }
        gelu16(lut, v, gv);
#pragma unroll
        for (int k = 0; k < 16; ++k) lds[lds_slot(16 * j + k)] = bf16_to_f32(gv[k]) * sn[k];
    }
    __syncthreads();
    rotate_quantize(lds, red, q, q4, ldq, scale, tok, N);
}

// Second half of a split gated-MLP middle: x = BF16(g * u) * su (g = GELU(gate), u = up, both BF16 (M, K)) -> walsh -> INT8.
__global__ void k_pre2(const u16* g, const u16* u, const i8* su, i8* q, int* q4, int ldq, float* scale, int K, int vec) {
    extern __shared__ float lds[];
    __shared__ float red[16];
    const int tok = blockIdx.x;
    const size_t base = (size_t)tok * K;
    for (int j = threadIdx.x; j < (K >> 4); j += blockDim.x) {
        float gv[16], uv[16], sn[16];
        c16_bf16(g + base + 16 * j, vec, gv);
        c16_bf16(u + base + 16 * j, vec, uv);
        c16_i8(su + 16 * j, vec, sn);
#pragma unroll
        for (int k = 0; k < 16; ++k) lds[lds_slot(16 * j + k)] = bf16_to_f32(f32_to_bf16(gv[k] * uv[k])) * sn[k];
    }
    for (int i = (K & ~15) + threadIdx.x; i < K; i += blockDim.x)        // widths that are not a multiple of 16
        lds[lds_slot(i)] = bf16_to_f32(f32_to_bf16(bf16_to_f32(gptr(g)[base + i]) * bf16_to_f32(gptr(u)[base + i]))) *
                           (float)gptr(su)[i];
    __syncthreads();
    rotate_quantize(lds, red, q, q4, ldq, scale, tok, K);
}

// --------------------------------------------------------------------------------------------- RMSNorm and its fusions
// Gemma RMSNorm with FP32 arithmetic and a BF16 result: y = bf16((x * r) * (1 + w)), r = 1 / sqrt(ss / K + eps), ss summed
// in the order of tree_total, so every kernel that normalises a row of width K gives the same bits. K % 16 == 0.
// The row is loaded (and its chunk sums taken) in one pass.
__device__ __forceinline__ void load_row_sumsq(float* lds, float* part, const u16* x, int K, bool vec) {
    for (int j = threadIdx.x; j < (K >> 4); j += blockDim.x) {
        float v[16];
        c16_bf16(x + 16 * j, vec, v);
#pragma unroll
        for (int k = 0; k < 16; ++k) lds[lds_slot(16 * j + k)] = v[k];
        part[j] = chunk_sumsq(v);
    }
    __syncthreads();
}

__global__ void k_rmsnorm(const u16* x, const u16* w, float eps, u16* y, int K, int vec) {
    extern __shared__ float lds[];
    __shared__ float red[16];
    float* part = lds + lds_words(K);
    const size_t base = (size_t)blockIdx.x * K;
    load_row_sumsq(lds, part, x + base, K, vec);
    norm_apply(lds, tree_total(part, red, K), w, nullptr, eps, K, vec);
    store_row<TCQ_BF16>(lds, y, base, K, vec, [](int, float(&)[8]) {}, [](int, float v) { return v; });
}

// RMSNorm -> * su -> block Walsh -> per-token INT8: the input norm of a decoder layer fused with the rotate + quantize
// prologue of the projections that read it.
__global__ void k_norm_pre(const u16* x, const u16* w, float eps, const i8* su, i8* q, int* q4, int ldq, float* scale, int K,
                           int vec) {
    extern __shared__ float lds[];
    __shared__ float red[16];
    float* part = lds + lds_words(K);
    const int tok = blockIdx.x, j0 = threadIdx.x;
    const bool has0 = j0 < (K >> 4);
    Raw16<2> w0{};
    Raw16<1> su0{};
    if (has0) {
        w0 = raw16<2>(w + 16 * j0, vec);
        if (su) su0 = raw16<1>(su + 16 * j0, vec);
    }
    load_row_sumsq(lds, part, x + (size_t)tok * K, K, vec);
    norm_apply(lds, tree_total(part, red, K), w, su, eps, K, vec, has0, w0, su0);
    rotate_quantize(lds, red, q, q4, ldq, scale, tok, K);
}

// Epilogue of a projection fused with the residual add and (w != NULL) the next norm + rotate + quantize:
// a = BF16(walsh(SCALE(acc)) * sv + bias); x_out = BF16(x + a); then, as k_norm_pre, q / scale of RMSNorm(x_out).
template <int ADT>
__global__ __launch_bounds__(512) void k_post_add_norm_pre(const void* acc, int lda, int col0, const float* s, const float* rs, const i8* sv,
                                    const float* bias, const u16* x, u16* xout, const u16* w, float eps, const i8* su, i8* q,
                                    int* q4, int ldq, float* scale, int N, int vec, int svec) {
    extern __shared__ float lds[];
    __shared__ float red[16];
    float* part = lds + lds_words(N);
    const int tok = blockIdx.x, j0 = threadIdx.x;
    const size_t row = (size_t)tok * N;
    const bool has0 = j0 < (N >> 4);
    Raw16<1> sv0{}, su0{};                                              // this thread's first chunk of every side vector
    Raw16<4> b0{};
    Raw16<2> x0{}, w0{};
    if (has0) {
        sv0 = raw16<1>(sv + 16 * j0, svec);
        if (bias) b0 = raw16<4>(bias + 16 * j0, svec);
        x0 = raw16<2>(x + row + 16 * j0, svec);
        if (w) w0 = raw16<2>(w + 16 * j0, svec);
        if (w && su) su0 = raw16<1>(su + 16 * j0, svec);
    }
    load_acc_row<ADT>(lds, acc, (size_t)tok * lda + col0, ADT == TCQ_I32 ? s[tok] : 1.f, rs, N, vec);
    walsh_inplace(lds, N);
    for (int j = j0; j < (N >> 4); j += blockDim.x) {
        float sg[16], b[16], xv[16];
        u16 xn[16];
        if (j == j0) {
            cv16(sv0, sg);
            if (bias) cv16(b0, b);
            cv16(x0, xv);
        } else {
            c16_i8(sv + 16 * j, svec, sg);
            if (bias) c16_f32(bias + 16 * j, svec, b);
            c16_bf16(x + row + 16 * j, svec, xv);
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            float v = lds[lds_slot(16 * j + k)] * sg[k];
            if (bias) v = v + b[k];
            xn[k] = f32_to_bf16(xv[k] + bf16_to_f32(f32_to_bf16(v)));
            xv[k] = bf16_to_f32(xn[k]);
            lds[lds_slot(16 * j + k)] = xv[k];
        }
        c16_store_bf16(xout + row + 16 * j, svec, xn);
        part[j] = chunk_sumsq(xv);
    }
    __syncthreads();
    if (!w) return;
    norm_apply(lds, tree_total(part, red, N), w, su, eps, N, svec, has0, w0, su0);
    rotate_quantize(lds, red, q, q4, ldq, scale, tok, N);
}

// k_postg for power-of-two segments of 256 .. 4096 on the register + transpose engine (16 values per thread; the workgroup
// has maxN / 16 threads, the threads past a narrower segment's count sit out), other segments through LDS as in k_postg:
// the same operations in the same order, y = conv(((walsh(acc) * c) * sv) (+ bias), GELU).
template <int ADT, int YDT, int L>
__device__ __forceinline__ void postg_tw_seg(const tcq_post_seg& S, int tok, float st, const u16* gelu, float* xs) {
    constexpr int N = 1 << L;
    const int t = threadIdx.x, i0 = 16 * t;
    const bool act = t < (N >> 4);
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = 0.f;
    Raw16<1> sv0{};
    Raw16<4> b0{};
    if (act) {
        sv0 = raw16<1>(S.sv + i0, true);
        if (S.bias) b0 = raw16<4>(S.bias + i0, true);
        acc_chunk<ADT>(S.acc, (size_t)tok * S.lda + S.col0 + i0, st, S.rs ? S.rs + i0 : nullptr, v);
    }
    tw_walsh<L, 4>(v, xs);
    const float c = (float)(1.0 / __builtin_sqrt((double)N));
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = v[k] * c;
    tw_to_natural<L, 4>(v, xs);
    if (!act) return;
    float sg[16], b[16];
    cv16(sv0, sg);
    if (S.bias) cv16(b0, b);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        v[k] = v[k] * sg[k];
        if (S.bias) v[k] = v[k] + b[k];
        if (YDT == TCQ_BF16 && gelu) v[k] = bf16_to_f32(gptr(gelu)[f32_to_bf16(v[k])]);
    }
    float a[8], bb[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) { a[k] = v[k]; bb[k] = v[8 + k]; }
    Elem<YDT>::st8(S.y, (size_t)tok * N + i0, a);
    Elem<YDT>::st8(S.y, (size_t)tok * N + i0 + 8, bb);
}

template <int ADT, int YDT, class SEGS>
__global__ void k_postg_tw(SEGS segs, const float* s, const u16* gelu_lut, int maxN) {
    extern __shared__ float lds[];
    const tcq_post_seg S = segs[blockIdx.y];
    const int tok = blockIdx.x, N = S.N;
    if (N <= 0 || N > maxN || (ADT != TCQ_F32 && !S.rs)) return;    // uniform
    const int esz = ADT == TCQ_BF16 ? 2 : 4, ysz = YDT == TCQ_F32 ? 4 : 2;
    const bool vec = N % 8 == 0 && aligned16(S.acc) && ((size_t)S.lda * esz) % 16 == 0 && ((size_t)S.col0 * esz) % 16 == 0 &&
                     aligned16(S.y) && ((size_t)N * ysz) % 16 == 0 && ((uintptr_t)S.sv & 7) == 0 && (!S.rs || aligned16(S.rs)) &&
                     (!S.bias || aligned16(S.bias));
    const float st = ADT == TCQ_I32 ? s[tok] : 1.f;
    const u16* gl = S.gelu ? gelu_lut : nullptr;
    if (vec && aligned16(S.sv)) {
        switch (N) {
            case 256: postg_tw_seg<ADT, YDT, 8>(S, tok, st, gl, lds); return;
            case 512: postg_tw_seg<ADT, YDT, 9>(S, tok, st, gl, lds); return;
            case 1024: postg_tw_seg<ADT, YDT, 10>(S, tok, st, gl, lds); return;
            case 2048: postg_tw_seg<ADT, YDT, 11>(S, tok, st, gl, lds); return;
            case 4096: postg_tw_seg<ADT, YDT, 12>(S, tok, st, gl, lds); return;
            default: break;
        }
    }
    load_acc_row<ADT>(lds, S.acc, (size_t)tok * S.lda + S.col0, st, S.rs, N, vec);
    walsh_inplace(lds, N);
    store_post_row<YDT>(lds, S.y, (size_t)tok * N, S.sv, S.bias, gl, N, vec);
}


// k_mid2 on the register + transpose engine for N = 2^L (2^LE values per thread, 2^(L - LE) threads, aligned): the gate half
// is loaded at entry and the up half during the gate's transform, each transform returns to the natural layout through LDS,
// so signs, GELU and rounding points are applied exactly as in k_mid2.
// At most 128 registers (4 waves per SIMD): two 512-thread rows of 16384 per CU, as their LDS allows (139 registers left one
// row per CU: 800 x 16384 72.4 -> 51.5 us on MI355X, bit-identical).
template <int ADT, int L, int LE>
__global__ __launch_bounds__(1 << (L - LE), 4) void k_mid2_tw(const void* acc, int lda, const float* s, const float* rs, const i8* sv,
                                                           const u16* lut, const i8* su, i8* q, int* q4, int ldq, float* scale) {
    constexpr int N = 1 << L, E = 1 << LE, NP = E / 16;
    extern __shared__ float xs[];
    __shared__ float red[16];
    const int tok = blockIdx.x, t = threadIdx.x, i0 = E * t;
    const size_t base = (size_t)tok * lda + i0;
    const float st = ADT == TCQ_I32 ? s[tok] : 1.f;
    Raw16<1> svg[NP], svu[NP], sn0[NP];
#pragma unroll
    for (int h = 0; h < NP; ++h) {
        svg[h] = raw16<1>(sv + i0 + 16 * h, true);
        svu[h] = raw16<1>(sv + N + i0 + 16 * h, true);
        sn0[h] = raw16<1>(su + i0 + 16 * h, true);
    }
    float g[E], u[E];
    // 4-byte accumulators: coalesced span loads staged through xs (the up half is loaded during the gate's transform and
    // staged after it); BF16: per-thread loads
    const u32* arow = (const u32*)acc + (size_t)tok * lda;
    Span<LE, 4> ga{}, ua{};
    auto stage = [&](const Span<LE, 4>& a, const float* r) {
        if (ADT == TCQ_I32) {
            // the scales' span in two halves, so that only half of it is live at a time
            const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
            const uint4_t* rp = (const uint4_t*)((const u32*)r + ((size_t)w << (LE + 6)));
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                uint4_t rv[E / 8];
#pragma unroll
                for (int j = 0; j < E / 8; ++j) rv[j] = *gptr(rp + 64 * (j + hh * E / 8) + lane);
#pragma unroll
                for (int j = 0; j < E / 8; ++j) {
                    const int jj = j + hh * E / 8;
                    float* d = xs + lds_slot((w << (LE + 6)) + 4 * (64 * jj + lane));
#pragma unroll
                    for (int m = 0; m < 4; ++m) d[m] = ((float)(int)a.p[jj][m] * st) * __uint_as_float(rv[j][m]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            tw_span_put<LE, 4>(a, xs, [&](int, int, u32 b) { return __uint_as_float(b); });
        }
        __syncthreads();
    };
    if constexpr (ADT == TCQ_BF16) {
#pragma unroll
        for (int h = 0; h < NP; ++h) {
            acc_chunk<ADT>(acc, base + 16 * h, st, rs + i0 + 16 * h, part16(g, h));
            acc_chunk<ADT>(acc, base + N + 16 * h, st, rs + N + i0 + 16 * h, part16(u, h));
        }
    } else {
        ga = tw_span_load<LE, 4>(arow);
        stage(ga, rs);
        ua = tw_span_load<LE, 4>(arow + N);      // after the barrier: in flight during the gate's transform
        tw_get<L, LE, 0>(g, xs);
    }
    const float c = (float)(1.0 / __builtin_sqrt((double)N));
    tw_walsh<L, LE>(g, xs);
    tw_to_natural<L, LE>(g, xs);
    u16x2_t gv[E / 2];                      // GELU values two per register (half-register gathers)
#pragma unroll
    for (int h = 0; h < NP; ++h) {
        float sg[16];
        cv16(svg[h], sg);
#pragma unroll
        for (int k = 0; k < 16; ++k) g[16 * h + k] = g[16 * h + k] * c * sg[k];
#pragma unroll
        for (int k = 0; k < 16; k += 2)
            gv[8 * h + k / 2] = u16x2_t{gptr(lut)[f32_to_bf16(g[16 * h + k])], gptr(lut)[f32_to_bf16(g[16 * h + k + 1])]};
    }
    if constexpr (ADT != TCQ_BF16) {
        stage(ua, rs ? rs + N : nullptr);     // writes only the wave's own span: its threads have finished reading it
        tw_get<L, LE, 0>(u, xs);
    }
    tw_walsh<L, LE>(u, xs);
    tw_to_natural<L, LE>(u, xs);
#pragma unroll
    for (int h = 0; h < NP; ++h) {
        float sgu[16], sn[16];
        cv16(svu[h], sgu);
        cv16(sn0[h], sn);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const float uu = bf16_to_f32(f32_to_bf16((u[16 * h + k] * c) * sgu[k]));
            u[16 * h + k] = bf16_to_f32(f32_to_bf16(bf16_to_f32(gv[8 * h + k / 2][k & 1]) * uu)) * sn[k];
        }
    }
    tw_rotate_quantize<L, LE>(u, xs, red, q, q4, ldq, scale, tok);
}

// k_postg_tw for groups whose segments are all 256 or 2048 wide, on the no-transpose engine with 4 values per thread:
// a 2048-wide segment on all 8 waves (one LDS exchange), a 256-wide one inside wave 0 (index bits inside the thread and
// across the lanes only). The same operations in the same order, y = conv(((walsh(acc) * c) * sv) (+ bias), GELU).
template <int ADT, int YDT, int L, int NWP>
__device__ __forceinline__ void postg_wv_seg(const tcq_post_seg& S, int tok, float st, const u16* gelu, float* xs) {
    constexpr int N = 1 << L;
    const int i0 = 4 * threadIdx.x;
    float v[4];
    const size_t base = (size_t)tok * S.lda + S.col0 + i0;
    if (ADT == TCQ_I32) {
        const uint4_t a = *gptr((const uint4_t*)((const u32*)S.acc + base));
        const float4_t r = *gptr((const float4_t*)(S.rs + i0));
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = ((float)(int)a[k] * st) * r[k];
    } else if (ADT == TCQ_BF16) {
        const uint2_t a = *gptr((const uint2_t*)((const u16*)S.acc + base));
        const float4_t r = *gptr((const float4_t*)(S.rs + i0));
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            v[2 * k] = __uint_as_float(a[k] << 16) * r[2 * k];
            v[2 * k + 1] = __uint_as_float(a[k] & 0xffff0000u) * r[2 * k + 1];
        }
    } else {
        const float4_t a = *gptr((const float4_t*)((const float*)S.acc + base));
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = a[k];
    }
    const u32 sg = *gptr((const u32*)(S.sv + i0));
    float4_t b = {0.f, 0.f, 0.f, 0.f};
    if (S.bias) b = *gptr((const float4_t*)(S.bias + i0));
    wave_walsh_lanes<2>(v);
    if constexpr (NWP > 1) {
        wave_walsh_put<2, NWP>(v, xs);
        __syncthreads();
        wave_walsh_get<2, NWP>(v, xs);
    }
    const float c = (float)(1.0 / __builtin_sqrt((double)N));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        v[k] = (v[k] * c) * (float)(i8)(sg >> (8 * k));
        if (S.bias) v[k] = v[k] + b[k];
        if (YDT == TCQ_BF16 && gelu) v[k] = bf16_to_f32(gptr(gelu)[f32_to_bf16(v[k])]);
    }
    const size_t o = (size_t)tok * N + i0;
    if constexpr (YDT == TCQ_F32) {
        *gptr((float4_t*)((float*)S.y + o)) = float4_t{v[0], v[1], v[2], v[3]};
    } else if constexpr (YDT == TCQ_BF16) {
        u32 w2[2];
        bf16_pack<2>(v, w2);
        *gptr((uint2_t*)((u16*)S.y + o)) = uint2_t{w2[0], w2[1]};
    } else {
        *gptr((uint2_t*)((u16*)S.y + o)) = uint2_t{(u32)f32_to_f16(v[0]) | ((u32)f32_to_f16(v[1]) << 16),
                                                   (u32)f32_to_f16(v[2]) | ((u32)f32_to_f16(v[3]) << 16)};
    }
}
// tcq_post of few rows 256 / 1024 / 2048 wide with 16-byte aligned operands on the no-transpose engine: one workgroup of
// 2^L / 256 waves per token (postg_wv_seg's steps).
template <int ADT, int YDT, int L, int NWP>
__global__ __launch_bounds__(64 * NWP) void k_post_wv(const void* acc, int lda, int col0, const float* s, const float* rs, const i8* sv,
                                                      const float* bias, void* y) {
    __shared__ float xs[NWP > 1 ? (1 << L) : 1];
    const tcq_post_seg S{acc, rs, sv, bias, y, lda, col0, 1 << L, 0};
    const int tok = blockIdx.x;
    postg_wv_seg<ADT, YDT, L, NWP>(S, tok, ADT == TCQ_I32 ? s[tok] : 1.f, nullptr, xs);
}

// Segments of other widths or alignments (device descriptors, which the host cannot inspect) take the LDS engine of
// k_postg (dynamic LDS of lds_words(maxN) floats).
template <int ADT, int YDT, class SEGS>
__global__ __launch_bounds__(512) void k_postg_wv(SEGS segs, const float* s, const u16* gelu_lut, int maxN) {
    extern __shared__ float lds[];
    __shared__ float xs[2048];
    const tcq_post_seg S = segs[blockIdx.y];
    const int tok = blockIdx.x, N = S.N;
    if (N <= 0 || N > maxN || (ADT != TCQ_F32 && !S.rs)) return;    // uniform
    const float st = ADT == TCQ_I32 ? s[tok] : 1.f;
    const u16* gl = S.gelu ? gelu_lut : nullptr;
    const int esz = ADT == TCQ_BF16 ? 2 : 4, ysz = YDT == TCQ_F32 ? 4 : 2;
    const bool al = aligned16(S.acc) && ((size_t)S.lda * esz) % 16 == 0 && ((size_t)S.col0 * esz) % 16 == 0 && aligned16(S.y) &&
                    aligned16(S.sv) && (!S.rs || aligned16(S.rs)) && (!S.bias || aligned16(S.bias));
    if (al && N == 2048) {                                           // uniform
        postg_wv_seg<ADT, YDT, 11, 8>(S, tok, st, gl, xs);
        return;
    }
    if (al && N == 256) {
        if (threadIdx.x < 64) postg_wv_seg<ADT, YDT, 8, 1>(S, tok, st, gl, xs);
        return;
    }
    const bool vec = N % 8 == 0 && al && ((size_t)N * ysz) % 16 == 0 && ((uintptr_t)S.sv & 7) == 0;
    load_acc_row<ADT>(lds, S.acc, (size_t)tok * S.lda + S.col0, st, S.rs, N, vec);
    walsh_inplace(lds, N);
    store_post_row<YDT>(lds, S.y, (size_t)tok * N, S.sv, S.bias, gl, N, vec);
}

// k_mid2 for few rows of 2^L = 1024 .. 4096 on the no-transpose engine: NWP waves, E = 2^L / 64 / NWP = 4 or 8 values of
// each half per thread (natural layout, loaded straight from the accumulators); the gate and up transforms share one LDS
// exchange (wave_walsh2), GELU, product and signs follow in the thread, then waves_rotate_quantize with its own exchange
// row. The same operations on each value in the same order as k_mid2_tw2.
template <int ADT, int L, int NWP>
__global__ __launch_bounds__(64 * NWP) void k_mid2_wv(const void* acc, int lda, const float* s, const float* rs, const i8* sv,
                                                      const u16* lut, const i8* su, i8* q, int* q4, int ldq, float* scale) {
    constexpr int N = 1 << L, E = N / 64 / NWP, LE = E == 8 ? 3 : 2;
    static_assert(E == 4 || E == 8, "4 or 8 values per thread");
    __shared__ float xg[N], xu[N];
    __shared__ WavesLdsN<N> Qr;
    const int tok = blockIdx.x, t = threadIdx.x, i0 = E * t;
    const size_t base = (size_t)tok * lda + i0;
    const float st = ADT == TCQ_I32 ? s[tok] : 1.f;
    auto ld_i8 = [&](const i8* p, float (&o)[E]) {
        if constexpr (E == 8) {
            ld8_i8v(p, o);
        } else {
            const u32 x = *gptr((const u32*)p);
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = (float)(i8)(x >> (8 * k));
        }
    };
    // accumulator values i0 .. i0 + E - 1 of the half at column offset h (scaled as acc_chunk scales them)
    auto ld_acc = [&](size_t off, const float* r, float (&o)[E]) {
        if constexpr (E == 8) {
            acc_piece8<ADT>(acc, base + off, st, r ? r + i0 : nullptr, o, 1, 0);
        } else if constexpr (ADT == TCQ_I32) {
            const uint4_t a = *gptr((const uint4_t*)((const u32*)acc + base + off));
            const float4_t rv = *gptr((const float4_t*)(r + i0));
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = ((float)(int)a[k] * st) * rv[k];
        } else if constexpr (ADT == TCQ_BF16) {
            const uint2_t a = *gptr((const uint2_t*)((const u16*)acc + base + off));
            const float4_t rv = *gptr((const float4_t*)(r + i0));
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                o[2 * k] = __uint_as_float(a[k] << 16) * rv[2 * k];
                o[2 * k + 1] = __uint_as_float(a[k] & 0xffff0000u) * rv[2 * k + 1];
            }
        } else {
            const float4_t a = *gptr((const float4_t*)((const float*)acc + base + off));
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = a[k];
        }
    };
    float g[E], u[E], sg[E], sgu[E], sn[E];
    ld_i8(sv + i0, sg);
    ld_i8(sv + N + i0, sgu);
    ld_i8(su + i0, sn);
    ld_acc(0, rs, g);
    ld_acc(N, rs ? rs + N : nullptr, u);
    const auto bar = [] { __syncthreads(); };
    const float c = (float)(1.0 / __builtin_sqrt((double)N));
    wave_walsh2<LE, NWP>(g, u, xg, xu, bar);
    u16 gv[E];
#pragma unroll
    for (int k = 0; k < E; ++k) gv[k] = gptr(lut)[f32_to_bf16(g[k] * c * sg[k])];
#pragma unroll
    for (int k = 0; k < E; ++k) {
        const float uu = bf16_to_f32(f32_to_bf16((u[k] * c) * sgu[k]));
        u[k] = bf16_to_f32(f32_to_bf16(bf16_to_f32(gv[k]) * uu)) * sn[k];
    }
    waves_rotate_quantize<NWP, L>(u, Qr, nullptr, nullptr, q, scale, bar, tok, q4, ldq);
}

// k_mid2_tw with the gate and up transforms side by side (tw_walsh2: one barrier per pass for both rows; LDS for two rows,
// so it serves as many rows as fit one wave of workgroups): the same operations on each row in the same order.
template <int ADT, int L, int LE>
__global__ __launch_bounds__(1 << (L - LE)) void k_mid2_tw2(const void* acc, int lda, const float* s, const float* rs, const i8* sv,
                                                            const u16* lut, const i8* su, i8* q, int* q4, int ldq, float* scale) {
    constexpr int N = 1 << L, E = 1 << LE, NP = E / 16;
    extern __shared__ float xs[];                                       // two lds_words(N) regions: gate, then up
    float* xu = xs + lds_words(N);
    __shared__ float red[16];
    const int tok = blockIdx.x, t = threadIdx.x, i0 = E * t;
    const size_t base = (size_t)tok * lda + i0;
    const float st = ADT == TCQ_I32 ? s[tok] : 1.f;
    Raw16<1> svg[NP], svu[NP], sn0[NP];
#pragma unroll
    for (int h = 0; h < NP; ++h) {
        svg[h] = raw16<1>(sv + i0 + 16 * h, true);
        svu[h] = raw16<1>(sv + N + i0 + 16 * h, true);
        sn0[h] = raw16<1>(su + i0 + 16 * h, true);
    }
    float g[E], u[E];
    if constexpr (ADT == TCQ_BF16) {
#pragma unroll
        for (int h = 0; h < NP; ++h) {
            acc_chunk<ADT>(acc, base + 16 * h, st, rs + i0 + 16 * h, part16(g, h));
            acc_chunk<ADT>(acc, base + N + 16 * h, st, rs + N + i0 + 16 * h, part16(u, h));
        }
    } else {
        const u32* arow = (const u32*)acc + (size_t)tok * lda;
        const Span<LE, 4> ga = tw_span_load<LE, 4>(arow), ua = tw_span_load<LE, 4>(arow + N);
        // 4-byte accumulators staged through LDS in natural order (int32: scaled as acc_chunk does, the scales' span in two
        // halves so that only half of it is live at a time)
        auto stage = [&](const Span<LE, 4>& a, const float* r, float* dst) {
            if (ADT == TCQ_I32) {
                const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
                const uint4_t* rp = (const uint4_t*)((const u32*)r + ((size_t)w << (LE + 6)));
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    uint4_t rv[E / 8];
#pragma unroll
                    for (int j = 0; j < E / 8; ++j) rv[j] = *gptr(rp + 64 * (j + hh * E / 8) + lane);
#pragma unroll
                    for (int j = 0; j < E / 8; ++j) {
                        const int jj = j + hh * E / 8;
                        float* d = dst + lds_slot((w << (LE + 6)) + 4 * (64 * jj + lane));
#pragma unroll
                        for (int m = 0; m < 4; ++m) d[m] = ((float)(int)a.p[jj][m] * st) * __uint_as_float(rv[j][m]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
                tw_span_put<LE, 4>(a, dst, [&](int, int, u32 b) { return __uint_as_float(b); });
            }
        };
        stage(ga, rs, xs);
        stage(ua, rs ? rs + N : nullptr, xu);
        __syncthreads();
        tw_get<L, LE, 0>(g, xs);
        tw_get<L, LE, 0>(u, xu);
    }
    const float c = (float)(1.0 / __builtin_sqrt((double)N));
    tw_walsh2<L, LE>(g, u, xs, xu);
    tw_to_natural2<L, LE>(g, u, xs, xu);
#pragma unroll
    for (int h = 0; h < NP; ++h) {
        float sg[16], sgu[16], sn[16];
        cv16(svg[h], sg);
        cv16(svu[h], sgu);
        cv16(sn0[h], sn);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const u16 gv = gptr(lut)[f32_to_bf16(g[16 * h + k] * c * sg[k])];
            const float uu = bf16_to_f32(f32_to_bf16((u[16 * h + k] * c) * sgu[k]));
            u[16 * h + k] = bf16_to_f32(f32_to_bf16(bf16_to_f32(gv) * uu)) * sn[k];
        }
    }
    tw_rotate_quantize<L, LE>(u, xs, red, q, q4, ldq, scale, tok);
}

// Register path of k_post_add_norm_pre for power-of-two rows of 256 .. 16384 (K / 16 threads, thread t owns chunk t, every
// pointer 16-byte aligned): the same operations in the same order, with the row in registers instead of LDS, the Walsh
// transforms on reg_walsh16 and every global load issued at entry.
template <int ADT>
__global__ __launch_bounds__(1024) void k_post_add_norm_pre_reg(const void* acc, int lda, int col0, const float* s, const float* rs,
                                                                const i8* sv, const float* bias, const u16* x, u16* xout, const u16* w,
                                                                float eps, const i8* su, i8* q, int* q4, int ldq, float* scale, int N,
                                                                int parts) {
    extern __shared__ float xs[];                                      // N floats: cross-wave exchange and chunk sums
    __shared__ float red[16];
    const int tok = blockIdx.x, t = threadIdx.x, i0 = 16 * t;
    const size_t row = (size_t)tok * N, base = (size_t)tok * lda + col0 + i0;
    // every global read of the thread, issued together
    const Raw16<1> sv0 = raw16<1>(sv + i0, true);
    const Raw16<2> x0 = raw16<2>(x + row + i0, true);
    Raw16<4> b0{};
    Raw16<2> w0{};
    Raw16<1> su0{};
    if (bias) b0 = raw16<4>(bias + i0, true);
    if (w) {
        w0 = raw16<2>(w + i0, true);
        su0 = raw16<1>(su + i0, true);
    }
    float v[16];
    acc_chunk<ADT>(acc, base, ADT == TCQ_I32 ? s[tok] : 1.f, rs ? rs + i0 : nullptr, v, parts, (size_t)gridDim.x * lda);
    const float c = (float)(1.0 / __builtin_sqrt((double)N));
    reg_walsh16(v, N, xs);
    float sg[16], b[16], xv[16];
    u16 xn[16];
    cv16(sv0, sg);
    if (bias) cv16(b0, b);
    cv16(x0, xv);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        float a = (v[k] * c) * sg[k];
        if (bias) a = a + b[k];
        xn[k] = f32_to_bf16(xv[k] + bf16_to_f32(f32_to_bf16(a)));
        xv[k] = bf16_to_f32(xn[k]);
    }
    c16_store_bf16(xout + row + i0, true, xn);
    if (!w) return;
    xs[t] = chunk_sumsq(xv);
    __syncthreads();
    const float ss = tree_total(xs, red, N);
    const float r = 1.f / __builtin_sqrtf(ss / (float)N + eps);
    float wv[16], sn[16];
    cv16(w0, wv);
    cv16(su0, sn);
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = bf16_to_f32(f32_to_bf16((xv[k] * r) * (1.f + wv[k]))) * sn[k];
    reg_rotate_quantize(v, N, xs, red, q, q4, ldq, scale, tok);
}

// k_post_add_norm_pre on the register + transpose engine for N = 2^L (2^LE values per thread, 2^(L - LE) >= 64 threads,
// every pointer 16-byte aligned): the same operations in the same order as k_post_add_norm_pre_reg; the row is in the
// natural layout for the epilogue, residual and norm (chunk sums of squares at chunk indices, summed by tree_total).
template <int ADT, int L, int LE>
__global__ __launch_bounds__(1 << (L - LE)) void k_post_add_norm_pre_tw(const void* acc, int lda, int col0, const float* s,
                                                                       const float* rs, const i8* sv, const float* bias, const u16* x,
                                                                       u16* xout, const u16* w, float eps, const i8* su, i8* q,
                                                                       int* q4, int ldq, float* scale, int parts) {
    extern __shared__ float xs[];                                      // lds_words(N) floats for the transposes, then N / 16 sums
    __shared__ float red[16];
    const PanpArgs A{acc, s, rs, sv, bias, x, xout, w, su, lda, col0, parts, (size_t)gridDim.x * lda, eps};
    float v[1 << LE];
    if (!panp_tw<ADT, L, LE>(A, blockIdx.x, true, v, xs, xs + lds_words(1 << L), red)) return;   // uniform
    tw_rotate_quantize<L, LE>(v, xs, red, q, q4, ldq, scale, blockIdx.x);
}

// k_post_add_norm_pre_tw for few rows of 1024 or 2048 with the norm and without bias, on the no-transpose engine
// (panp_waves, waves_rotate_quantize): NWP waves per row, 4 values per thread, one LDS exchange per transform; the same
// values as k_post_add_norm_pre_tw.
template <int ADT, int L, int NWP>
__global__ __launch_bounds__(64 * NWP) void k_post_add_norm_pre_wv(const void* acc, int lda, int col0, const float* s,
                                                                  const float* rs, const i8* sv, const u16* x, u16* xout,
                                                                  const u16* w, float eps, const i8* su, i8* q, int* q4, int ldq,
                                                                  float* scale, int parts) {
    __shared__ WavesLds Q;
    const PanpArgs A{acc, s, rs, sv, nullptr, x, xout, w, su, lda, col0, parts, (size_t)gridDim.x * lda, eps};
    float v[(1 << L) / 64 / NWP];
    const auto bar = [] { __syncthreads(); };
    panp_waves<ADT, NWP, L>(A, blockIdx.x, true, v, Q, NoMid{}, bar);
    waves_rotate_quantize<NWP, L>(v, Q, nullptr, nullptr, q, scale, bar, blockIdx.x, q4, ldq);
}

// =========================================================================================================== C ABI
// Threads per row: few rows (latency) -> about one 8-element vector per thread (up to 1024 threads when there are fewer
// rows than CUs); many rows (throughput) -> four vectors per thread so more rows share a CU. Every row kernel's result is
// independent of the thread count.
static int row_threads(int M, int K) {
    const int per = M <= 256 ? 8 : 32;
    const int cap = M <= 64 ? 1024 : 512;        // fewer rows than CUs: wide rows take whole 1024-thread workgroups
    int t = 64;
    while (t < cap && t * per < K) t <<= 1;
    return t;
}
static size_t row_lds(int K) { return (size_t)lds_words(K) * sizeof(float); }
static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }
static bool al8(const void* p) { return ((uintptr_t)p & 7) == 0; }
// q4 output: the (K / 4, ldq >= M) word layout, or the token-block layout (ldq == TCQ_LDQ_TOKEN_BLOCKS)
static bool q4_bad(const void* q4, int ldq, int M) { return q4 && ldq != TCQ_LDQ_TOKEN_BLOCKS && ldq < M; }
static bool q4_tb_shape_bad(const void* q4, int ldq, int K) { return q4 && ldq == TCQ_LDQ_TOKEN_BLOCKS && K % 16; }
static int dsize(int dt) { return dt == TCQ_F32 || dt == TCQ_I32 ? 4 : dt == TCQ_I8 ? 1 : 2; }

#define DISPATCH_X(dt, KERNEL, ...)                                                             \
    switch (dt) {                                                                               \
        case TCQ_F32: { KERNEL(TCQ_F32, __VA_ARGS__); break; }                                  \
        case TCQ_BF16: { KERNEL(TCQ_BF16, __VA_ARGS__); break; }                                \
        case TCQ_F16: { KERNEL(TCQ_F16, __VA_ARGS__); break; }                                  \
        default: return TCQ_ERR_DTYPE;                                                          \
    }

template <int XD, int YD>
static void launch_rht_tw(int n, int M, hipStream_t st, const void* x, int ldx, const i8* su, void* y, int ldy) {
    const size_t sh = (size_t)lds_words(n) * sizeof(float);
    if (n == 1024) launch_k(k_rht_tw<XD, YD, 10, 4>, dim3(M), dim3(64), sh, st, x, ldx, su, y, ldy);
    else if (n == 2048) launch_k(k_rht_tw<XD, YD, 11, 4>, dim3(M), dim3(128), sh, st, x, ldx, su, y, ldy);
    else if (n == 4096) launch_k(k_rht_tw<XD, YD, 12, 4>, dim3(M), dim3(256), sh, st, x, ldx, su, y, ldy);
    else if (n == 8192) launch_k(k_rht_tw<XD, YD, 13, 5>, dim3(M), dim3(256), sh, st, x, ldx, su, y, ldy);
    else launch_k(k_rht_tw<XD, YD, 14, 5>, dim3(M), dim3(512), sh, st, x, ldx, su, y, ldy);
}

extern "C" int tcq_rht(const void* x, int x_dtype, int ldx, const int8_t* su, void* y, int y_dtype, int ldy, int M, int n,
                       tcq_stream_t stream) {
    if (!x || !y || M <= 0 || n <= 0 || ldx < n || ldy < n) return TCQ_ERR_ARG;
    if (n > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    const dim3 grid(M), block(row_threads(M, n));
    const size_t sh = row_lds(n);
    const int vec = n % 8 == 0 && al16(x) && al16(y) && ((size_t)ldx * dsize(x_dtype)) % 16 == 0 &&
                    ((size_t)ldy * dsize(y_dtype)) % 16 == 0 && (!su || al8(su));
    hipStream_t st = (hipStream_t)stream;
    // register + transpose engine for power-of-two rows of 1024 .. 16384
    if ((n & (n - 1)) == 0 && n >= 1024 && vec && (!su || al16(su))) {
#define RHT_Y(XD, YD) launch_rht_tw<XD, YD>(n, M, st, x, ldx, (const i8*)su, y, ldy)
#define RHT_X(XD, _)                                          \
    switch (y_dtype) {                                        \
        case TCQ_F32: RHT_Y(XD, TCQ_F32); break;              \
        case TCQ_BF16: RHT_Y(XD, TCQ_BF16); break;            \
        case TCQ_F16: RHT_Y(XD, TCQ_F16); break;              \
        default: return TCQ_ERR_DTYPE;                        \
    }
        DISPATCH_X(x_dtype, RHT_X, 0)
#undef RHT_X
#undef RHT_Y
        return launch_status();
    }
#define RHT_Y(XD, YD) launch_k(k_rht<XD, YD>, grid, block, sh, st, x, ldx, (const i8*)su, y, ldy, n, vec)
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

extern "C" int tcq_pre_h(const void* x, int x_dtype, const int8_t* su, uint16_t* h, uint16_t* hT, int ldh, int M, int K,
                         tcq_stream_t stream) {
    if (!x || (!h && !hT) || M <= 0 || K <= 0 || (hT && ldh < M)) return TCQ_ERR_ARG;
    if (K > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    if (hT && (size_t)K * ldh >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
    if (!hT) return tcq_rht(x, x_dtype, K, su, h, TCQ_BF16, K, M, K, stream);      // row-major only: the rotation engines
    const dim3 grid(M), block(row_threads(M, K));
    const int vec = K % 8 == 0 && al16(x) && ((size_t)K * dsize(x_dtype)) % 16 == 0 && (!su || al8(su));
    hipStream_t st = (hipStream_t)stream;
#define PREH(XD, _) launch_k(k_pre_hT<XD>, grid, block, row_lds(K), st, x, (const i8*)su, (u16*)h, (u16*)hT, K, ldh, vec)
    DISPATCH_X(x_dtype, PREH, 0)
#undef PREH
    return launch_status();
}

extern "C" int tcq_mid2_available(int N) { return N > 0 && N % 16 == 0 && N <= TCQ_MAX_WIDTH; }

extern "C" int tcq_pre_cs(const void* x, int x_dtype, const int8_t* su, const void* col_scale, int8_t* q, int32_t* q4, int ldq,
                          float* scale, int M, int K, tcq_stream_t stream) {
    if (!x || !scale || (!q && !q4) || M <= 0 || K <= 0 || q4_bad(q4, ldq, M)) return TCQ_ERR_ARG;
    if (K % 4 || K > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    if (q4_tb_shape_bad(q4, ldq, K)) return TCQ_ERR_SHAPE;
    if (q4 && ldq == TCQ_LDQ_TOKEN_BLOCKS && !al16(q4)) return TCQ_ERR_ALIGN;
    const dim3 grid(M), block(row_threads(M, K));
    const size_t sh = row_lds(K);
    const int vec = K % 8 == 0 && al16(x) && ((size_t)K * dsize(x_dtype)) % 16 == 0 && (!su || al8(su));
    hipStream_t st = (hipStream_t)stream;
    const u16* cs = (const u16*)col_scale;
    // register + transpose engine: power-of-two rows of 1024 .. 16384 without column scales, aligned
    if (!cs && (K & (K - 1)) == 0 && K >= 1024 && al16(x) && (!su || al16(su)) && (!q || al16(q)) &&
        (!q4 || ldq != TCQ_LDQ_TOKEN_BLOCKS || al16(q4))) {
        const size_t tsh = (size_t)lds_words(K) * sizeof(float);
        i8* qq = (i8*)q;
        int* q4p = (int*)q4;
        const i8* sp = (const i8*)su;
#define PRE_TW(XD, L, LE, T) launch_k(k_pre_tw<XD, L, LE>, grid, dim3(T), tsh, st, x, sp, qq, q4p, ldq, scale)
#define PRE_TWX(XD, _)                                                        \
    switch (K) {                                                              \
        case 1024: PRE_TW(XD, 10, 4, 64); break;                              \
        case 2048: PRE_TW(XD, 11, 4, 128); break;                             \
        case 4096: PRE_TW(XD, 12, 4, 256); break;                             \
        case 8192: PRE_TW(XD, 13, 5, 256); break;                             \
        default: PRE_TW(XD, 14, 5, 512); break;                               \
    }
        DISPATCH_X(x_dtype, PRE_TWX, 0)
#undef PRE_TWX
#undef PRE_TW
        return launch_status();
    }
#define PRE(XD, _) launch_k(k_pre<XD>, grid, block, sh, st, x, (const i8*)su, (i8*)q, (int*)q4, ldq, scale, K, vec, cs)
    DISPATCH_X(x_dtype, PRE, 0)
#undef PRE
    return launch_status();
}

extern "C" int tcq_pre(const void* x, int x_dtype, const int8_t* su, int8_t* q, int32_t* q4, int ldq, float* scale, int M, int K,
                       tcq_stream_t stream) {
    return tcq_pre_cs(x, x_dtype, su, nullptr, q, q4, ldq, scale, M, K, stream);
}

extern "C" int tcq_pre_h16(const void* x, int x_dtype, const int8_t* su, void* h16, float* hscale, int M, int K,
                           tcq_stream_t stream) {
    if (!x || !h16 || !hscale || M <= 0 || K <= 0) return TCQ_ERR_ARG;
    if (K > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    const dim3 grid(M), block(row_threads(M, K));
    const size_t sh = row_lds(K);
    const int vec = K % 8 == 0 && al16(x) && al16(h16) && ((size_t)K * dsize(x_dtype)) % 16 == 0 && (!su || al8(su));
    hipStream_t st = (hipStream_t)stream;
    if (M <= 64 && (K == 1024 || K == 2048) && vec && (!su || al16(su))) {   // few rows: the no-transpose engine
#define PREHW(XD, _) if (K == 1024) launch_k(k_pre_h16_wv<XD, 10, 4>, grid, dim3(256), 0, st, x, (const i8*)su, (u16*)h16, hscale); \
                     else launch_k(k_pre_h16_wv<XD, 11, 8>, grid, dim3(512), 0, st, x, (const i8*)su, (u16*)h16, hscale)
        DISPATCH_X(x_dtype, PREHW, 0)
#undef PREHW
        return launch_status();
    }
    if ((K & (K - 1)) == 0 && K >= 256 && vec && (!su || al16(su))) {     // register engine
        const int nt = K / 16 < 64 ? 64 : K / 16;
#define PREHR(XD, _) launch_k(k_pre_h16_reg<XD>, grid, dim3(nt), (size_t)K * sizeof(float), st, x, (const i8*)su, (u16*)h16, hscale, K)
        DISPATCH_X(x_dtype, PREHR, 0)
#undef PREHR
        return launch_status();
    }
#define PREH(XD, _) launch_k(k_pre_h16<XD>, grid, block, sh, st, x, (const i8*)su, (u16*)h16, hscale, K, vec)
    DISPATCH_X(x_dtype, PREH, 0)
    return launch_status();
}

extern "C" int tcq_quantize_rows(const void* x, int x_dtype, int ldx, int8_t* q, float* scale, int M, int K, tcq_stream_t stream) {
    if (!x || !q || !scale || M <= 0 || K <= 0 || ldx < K) return TCQ_ERR_ARG;
    if (K % 4 || K > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    const dim3 grid(M), block(row_threads(M, K));
    const size_t sh = row_lds(K);
    const int vec = K % 8 == 0 && al16(x) && ((size_t)ldx * dsize(x_dtype)) % 16 == 0;
    hipStream_t st = (hipStream_t)stream;
#define QROWS(XD, _) launch_k(k_quantize_rows<XD>, grid, block, sh, st, x, ldx, (i8*)q, scale, K, vec)
    DISPATCH_X(x_dtype, QROWS, 0)
    return launch_status();
}

// Epilogue of a one-sided layer (no output rotation, the GR00T "tcq" base): y[t, i] = SCALE(acc[t, col0 + i]) (+ bias[i]),
// SCALE as in k_post. grid (ceil(N / 256), M), one element per thread.
template <int ADT, int YDT>
__global__ __launch_bounds__(256) void k_post_plain(const void* acc, int lda, int col0, const float* s, const float* rs,
                                                    const float* bias, void* y, int N) {
    const int i = blockIdx.x * 256 + threadIdx.x, tok = blockIdx.y;
    if (i >= N) return;
    const size_t a = (size_t)tok * lda + col0 + i;
    float z;
    if constexpr (ADT == TCQ_I32) z = ((float)gptr((const int*)acc)[a] * gptr(s)[tok]) * gptr(rs)[i];
    else if constexpr (ADT == TCQ_BF16) z = bf16_to_f32(gptr((const u16*)acc)[a]) * gptr(rs)[i];
    else z = gptr((const float*)acc)[a];
    if (bias) z = z + gptr(bias)[i];
    const size_t o = (size_t)tok * N + i;
    if constexpr (YDT == TCQ_F32) gptr((float*)y)[o] = z;
    else if constexpr (YDT == TCQ_BF16) gptr((u16*)y)[o] = f32_to_bf16(z);
    else gptr((u16*)y)[o] = f32_to_f16(z);
}

extern "C" int tcq_post(const void* acc, int acc_dtype, int lda, int col0, const float* s, const float* rs, const int8_t* sv,
                        const float* bias, void* y, int y_dtype, int M, int N, tcq_stream_t stream) {
    if (!acc || !y || M <= 0 || N <= 0 || col0 < 0 || lda < col0 + N) return TCQ_ERR_ARG;
    if ((acc_dtype == TCQ_I32 && (!s || !rs)) || (acc_dtype == TCQ_BF16 && !rs)) return TCQ_ERR_ARG;
    if (!sv) {                                                   // one-sided layer: no output rotation
        const dim3 grid((N + 255) / 256, M);
        hipStream_t st = (hipStream_t)stream;
#define PLAIN_Y(AD, YD) launch_k(k_post_plain<AD, YD>, grid, dim3(256), 0, st, acc, lda, col0, s, rs, bias, y, N)
#define PLAIN_A(AD)                                          \
    switch (y_dtype) {                                       \
        case TCQ_F32: PLAIN_Y(AD, TCQ_F32); break;           \
        case TCQ_BF16: PLAIN_Y(AD, TCQ_BF16); break;         \
        case TCQ_F16: PLAIN_Y(AD, TCQ_F16); break;           \
        default: return TCQ_ERR_DTYPE;                       \
    }
        switch (acc_dtype) {
            case TCQ_I32: PLAIN_A(TCQ_I32); break;
            case TCQ_F32: PLAIN_A(TCQ_F32); break;
            case TCQ_BF16: PLAIN_A(TCQ_BF16); break;
            default: return TCQ_ERR_DTYPE;
        }
#undef PLAIN_A
#undef PLAIN_Y
        return launch_status();
    }
    if (N > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    const int asz = dsize(acc_dtype);
    if (M <= 64 && (N == 256 || N == 1024 || N == 2048) && al16(acc) && ((size_t)lda * asz) % 16 == 0 && ((size_t)col0 * asz) % 16 == 0 &&
        al16(y) && al16(sv) && (!rs || al16(rs)) && (!bias || al16(bias))) {   // few rows: the no-transpose engine
        hipStream_t st = (hipStream_t)stream;
#define POSTW_K(AD, YD, L, NWP) launch_k(k_post_wv<AD, YD, L, NWP>, dim3(M), dim3(64 * NWP), 0, st, acc, lda, col0, s, rs, (const i8*)sv, bias, y)
#define POSTW_Y(AD, YD)                                                                                                    \
    if (N == 2048) POSTW_K(AD, YD, 11, 8);                                                                                 \
    else if (N == 1024) POSTW_K(AD, YD, 10, 4);                                                                            \
    else POSTW_K(AD, YD, 8, 1)
#define POSTW_A(AD)                                          \
    switch (y_dtype) {                                       \
        case TCQ_F32: POSTW_Y(AD, TCQ_F32); break;           \
        case TCQ_BF16: POSTW_Y(AD, TCQ_BF16); break;         \
        case TCQ_F16: POSTW_Y(AD, TCQ_F16); break;           \
        default: return TCQ_ERR_DTYPE;                       \
    }
        switch (acc_dtype) {
            case TCQ_I32: POSTW_A(TCQ_I32); break;
            case TCQ_F32: POSTW_A(TCQ_F32); break;
            case TCQ_BF16: POSTW_A(TCQ_BF16); break;
            default: return TCQ_ERR_DTYPE;
        }
#undef POSTW_A
#undef POSTW_Y
#undef POSTW_K
        return launch_status();
    }
    const dim3 grid(M), block(row_threads(M, N));
    const size_t sh = row_lds(N);
    const int vec = N % 8 == 0 && al16(acc) && ((size_t)lda * asz) % 16 == 0 && ((size_t)col0 * asz) % 16 == 0 && al16(y) &&
                    ((size_t)N * dsize(y_dtype)) % 16 == 0 && al8(sv) && (!rs || al16(rs)) && (!bias || al16(bias));
    hipStream_t st = (hipStream_t)stream;
#define POST_Y(AD, YD) launch_k(k_post<AD, YD>, grid, block, sh, st, acc, lda, col0, s, rs, (const i8*)sv, bias, y, N, vec)
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
    const bool tw = (maxN & (maxN - 1)) == 0 && maxN >= 256 && maxN <= 4096;
    const bool wv = M <= 64 && maxN == 2048;                 // few tokens: 2048 / 256-wide segments on the no-transpose engine
    const dim3 grid(M, nseg), block(wv ? 512 : tw ? maxN / 16 : row_threads(M * nseg, maxN));
    const size_t sh = row_lds(maxN);
    hipStream_t st = (hipStream_t)stream;
#define POSTG_Y(AD, YD)                                                                                                    \
    if (wv) launch_k(k_postg_wv<AD, YD, const tcq_post_seg*>, grid, block, sh, st, segs, s, (const u16*)gelu_lut, maxN);   \
    else if (tw) launch_k(k_postg_tw<AD, YD, const tcq_post_seg*>, grid, block, sh, st, segs, s, (const u16*)gelu_lut, maxN); \
    else launch_k(k_postg<AD, YD, const tcq_post_seg*>, grid, block, sh, st, segs, s, (const u16*)gelu_lut, maxN)
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

extern "C" int tcq_mid2(const void* acc, int acc_dtype, int lda, const float* s, const float* rs, const int8_t* sv,
                        const uint16_t* gelu_lut, const int8_t* su, int8_t* q, int32_t* q4, int ldq, float* scale, int M, int N,
                        tcq_stream_t stream) {
    if (!acc || !sv || !gelu_lut || !su || !scale || (!q && !q4) || M <= 0 || N <= 0 || lda < 2 * N || q4_bad(q4, ldq, M))
        return TCQ_ERR_ARG;
    if ((acc_dtype == TCQ_I32 && (!s || !rs)) || (acc_dtype == TCQ_BF16 && !rs)) return TCQ_ERR_ARG;
    if (N % 16 || N > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    if (q4_tb_shape_bad(q4, ldq, N)) return TCQ_ERR_SHAPE;
    if (q4 && ldq == TCQ_LDQ_TOKEN_BLOCKS && !al16(q4)) return TCQ_ERR_ALIGN;
    const dim3 grid(M), block(row_threads(M, N));
    const size_t sh = row_lds(N) + (size_t)N * 2;
    const int asz = dsize(acc_dtype);
    const int vec = al16(acc) && ((size_t)lda * asz) % 16 == 0 && (!rs || al16(rs));
    const int svec = al16(sv) && al16(su);
    hipStream_t st = (hipStream_t)stream;
    const i8 *svp = (const i8*)sv, *sup = (const i8*)su;
    // register + transpose engine: power-of-two widths 2^10 .. 2^14 (16 values of each half per thread up to 4096, 32 beyond;
    // measured on MI355X: 50 x 4096 in 7.5 us against 9.8 with 32 and 11.3 on the register engine), aligned
    if (N >= 1024 && (N & (N - 1)) == 0 && vec && svec && (!q || al16(q))) {
        const size_t tsh = (size_t)lds_words(N) * sizeof(float);
#define MID2_TWK(KER, L, LE, SH)                                                                                             \
    switch (acc_dtype) {                                                                                                      \
        case TCQ_I32: launch_k(KER<TCQ_I32, L, LE>, grid, dim3(1 << (L - LE)), SH, st, acc, lda, s, rs, svp, gelu_lut, sup,      \
                               (i8*)q, (int*)q4, ldq, scale); break;                                                          \
        case TCQ_F32: launch_k(KER<TCQ_F32, L, LE>, grid, dim3(1 << (L - LE)), SH, st, acc, lda, s, rs, svp, gelu_lut, sup,      \
                               (i8*)q, (int*)q4, ldq, scale); break;                                                          \
        case TCQ_BF16: launch_k(KER<TCQ_BF16, L, LE>, grid, dim3(1 << (L - LE)), SH, st, acc, lda, s, rs, svp, gelu_lut, sup,    \
                                (i8*)q, (int*)q4, ldq, scale); break;                                                         \
        default: return TCQ_ERR_DTYPE;                                                                                        \
    }
        if (M <= 64 && N <= 4096) {                       // few rows: the no-transpose engine on 4 (1024) or 8 waves
#define MID2_WV(L, NWP)                                                                                                     \
    switch (acc_dtype) {                                                                                                      \
        case TCQ_I32: launch_k(k_mid2_wv<TCQ_I32, L, NWP>, grid, dim3(64 * NWP), 0, st, acc, lda, s, rs, svp, gelu_lut, sup,     \
                               (i8*)q, (int*)q4, ldq, scale); break;                                                          \
        case TCQ_F32: launch_k(k_mid2_wv<TCQ_F32, L, NWP>, grid, dim3(64 * NWP), 0, st, acc, lda, s, rs, svp, gelu_lut, sup,     \
                               (i8*)q, (int*)q4, ldq, scale); break;                                                          \
        case TCQ_BF16: launch_k(k_mid2_wv<TCQ_BF16, L, NWP>, grid, dim3(64 * NWP), 0, st, acc, lda, s, rs, svp, gelu_lut, sup,   \
                                (i8*)q, (int*)q4, ldq, scale); break;                                                         \
        default: return TCQ_ERR_DTYPE;                                                                                        \
    }
            if (N == 1024) MID2_WV(10, 4)
            else if (N == 2048) MID2_WV(11, 8)
            else MID2_WV(12, 8)
#undef MID2_WV
            return launch_status();
        }
        if (M <= 256) {                                   // gate and up side by side (two LDS rows per workgroup)
#undef MID2_TW
#define MID2_TW(L, LE) MID2_TWK(k_mid2_tw2, L, LE, 2 * tsh)
            if (N == 1024) MID2_TW(10, 4)
            else if (N == 2048) MID2_TW(11, 4)
            else if (N == 4096) MID2_TW(12, 4)
            else if (N == 8192) MID2_TW(13, 5)
            else MID2_TW(14, 5)
            return launch_status();
        }
#undef MID2_TW
#define MID2_TW(L, LE) MID2_TWK(k_mid2_tw, L, LE, tsh)
        if (N == 1024) MID2_TW(10, 4)
        else if (N == 2048) MID2_TW(11, 4)
        else if (N == 4096) MID2_TW(12, 4)
        else if (N == 8192) MID2_TW(13, 5)
        else MID2_TW(14, 5)
#undef MID2_TW
#undef MID2_TWK
        return launch_status();
    }
    switch (acc_dtype) {
        case TCQ_I32: launch_k(k_mid2<TCQ_I32>, grid, block, sh, st, acc, lda, s, rs, svp, gelu_lut, sup, (i8*)q, (int*)q4, ldq, scale, N, vec, svec); break;
        case TCQ_F32: launch_k(k_mid2<TCQ_F32>, grid, block, sh, st, acc, lda, s, rs, svp, gelu_lut, sup, (i8*)q, (int*)q4, ldq, scale, N, vec, svec); break;
        case TCQ_BF16: launch_k(k_mid2<TCQ_BF16>, grid, block, sh, st, acc, lda, s, rs, svp, gelu_lut, sup, (i8*)q, (int*)q4, ldq, scale, N, vec, svec); break;
        default: return TCQ_ERR_DTYPE;
    }
    return launch_status();
}

extern "C" int tcq_mid1(const void* acc, int acc_dtype, int lda, const float* s, const float* rs, const int8_t* sv, const float* bias,
                        const uint16_t* gelu_lut, const int8_t* su, int8_t* q, int32_t* q4, int ldq, float* scale, int M, int N,
                        tcq_stream_t stream) {
    if (!acc || !sv || !gelu_lut || !su || !scale || (!q && !q4) || M <= 0 || N <= 0 || lda < N || q4_bad(q4, ldq, M))
        return TCQ_ERR_ARG;
    if ((acc_dtype == TCQ_I32 && (!s || !rs)) || (acc_dtype == TCQ_BF16 && !rs)) return TCQ_ERR_ARG;
    if (N % 16 || N > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    if (q4_tb_shape_bad(q4, ldq, N)) return TCQ_ERR_SHAPE;
    if (q4 && ldq == TCQ_LDQ_TOKEN_BLOCKS && !al16(q4)) return TCQ_ERR_ALIGN;
    const dim3 grid(M), block(row_threads(M, N));
    const size_t sh = row_lds(N);
    const int asz = dsize(acc_dtype);
    const int vec = al16(acc) && ((size_t)lda * asz) % 16 == 0 && (!rs || al16(rs));
    const int svec = al16(sv) && al16(su) && (!bias || al16(bias));
    hipStream_t st = (hipStream_t)stream;
    const i8 *svp = (const i8*)sv, *sup = (const i8*)su;
    switch (acc_dtype) {
        case TCQ_I32: launch_k(k_mid1<TCQ_I32>, grid, block, sh, st, acc, lda, s, rs, svp, bias, gelu_lut, sup, (i8*)q, (int*)q4, ldq, scale, N, vec, svec); break;
        case TCQ_F32: launch_k(k_mid1<TCQ_F32>, grid, block, sh, st, acc, lda, s, rs, svp, bias, gelu_lut, sup, (i8*)q, (int*)q4, ldq, scale, N, vec, svec); break;
        case TCQ_BF16: launch_k(k_mid1<TCQ_BF16>, grid, block, sh, st, acc, lda, s, rs, svp, bias, gelu_lut, sup, (i8*)q, (int*)q4, ldq, scale, N, vec, svec); break;
        default: return TCQ_ERR_DTYPE;
    }
    return launch_status();
}

extern "C" int tcq_pre2(const void* g, const void* u, const int8_t* su, int8_t* q, int32_t* q4, int ldq, float* scale, int M, int K,
                        tcq_stream_t stream) {
    if (!g || !u || !su || !scale || (!q && !q4) || M <= 0 || K <= 0 || q4_bad(q4, ldq, M)) return TCQ_ERR_ARG;
    if (K % 4 || K > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    if (q4_tb_shape_bad(q4, ldq, K)) return TCQ_ERR_SHAPE;
    if (q4 && ldq == TCQ_LDQ_TOKEN_BLOCKS && !al16(q4)) return TCQ_ERR_ALIGN;
    const int vec = K % 8 == 0 && al16(g) && al16(u) && al16(su);
    launch_k(k_pre2, dim3(M), dim3(row_threads(M, K)), row_lds(K), (hipStream_t)stream, (const u16*)g, (const u16*)u, (const i8*)su,
             (i8*)q, (int*)q4, ldq, scale, K, vec);
    return launch_status();
}

extern "C" int tcq_post_group(const tcq_post_seg* segs, int nseg, int acc_dtype, const float* s, const uint16_t* gelu_lut, int y_dtype,
                              int M, tcq_stream_t stream) {
    if (!segs || nseg <= 0 || M <= 0) return TCQ_ERR_ARG;
    if (nseg > TCQ_MAX_SEGS) return TCQ_ERR_UNSUPPORTED;
    if (acc_dtype == TCQ_I32 && !s) return TCQ_ERR_ARG;
    PostPack pk;
    int maxN = 0;
    for (int i = 0; i < nseg; ++i) {
        const tcq_post_seg& g = segs[i];
        if (!g.acc || !g.sv || !g.y || g.N <= 0 || g.col0 < 0 || g.lda < g.col0 + g.N) return TCQ_ERR_ARG;
        if (acc_dtype != TCQ_F32 && !g.rs) return TCQ_ERR_ARG;
        if (g.gelu && (!gelu_lut || y_dtype != TCQ_BF16)) return TCQ_ERR_ARG;
        pk.s[i] = g;
        maxN = g.N > maxN ? g.N : maxN;
    }
    for (int i = nseg; i < TCQ_MAX_SEGS; ++i) pk.s[i] = tcq_post_seg{};
    if (maxN > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    // widest segment a power of two of 256 .. 4096: the register + transpose engine (16 values per thread) for the
    // power-of-two segments; measured on MI355X for q / k / v of 2048 / 256 / 256 at 50 tokens: 3.5 us against 4.1 on LDS
    const bool tw = (maxN & (maxN - 1)) == 0 && maxN >= 256 && maxN <= 4096;
    // few tokens and segments of 256 / 2048 only, 16-byte aligned: the no-transpose engine (k_postg_wv)
    const int esz = dsize(acc_dtype), ysz = dsize(y_dtype);
    bool wv = M <= 64;
    for (int i = 0; i < nseg; ++i) {
        const tcq_post_seg& g = segs[i];
        wv = wv && (g.N == 256 || g.N == 2048) && al16(g.acc) && ((size_t)g.lda * esz) % 16 == 0 && ((size_t)g.col0 * esz) % 16 == 0 &&
             al16(g.y) && al16(g.sv) && (!g.rs || al16(g.rs)) && (!g.bias || al16(g.bias)) && ysz >= 2;
    }
    const dim3 grid(M, nseg), block(wv ? 512 : tw ? maxN / 16 : row_threads(M * nseg, maxN));
    // no dynamic LDS for k_postg_wv here: its own checks equal the ones above, so it never takes its LDS fallback
    const size_t sh = wv ? 0 : row_lds(maxN);
    hipStream_t st = (hipStream_t)stream;
#define POSTV_Y(AD, YD)                                                                                                    \
    if (wv) launch_k(k_postg_wv<AD, YD, PostPack>, grid, block, sh, st, pk, s, (const u16*)gelu_lut, maxN);                \
    else if (tw) launch_k(k_postg_tw<AD, YD, PostPack>, grid, block, sh, st, pk, s, (const u16*)gelu_lut, maxN);           \
    else launch_k(k_postg<AD, YD, PostPack>, grid, block, sh, st, pk, s, (const u16*)gelu_lut, maxN)
#define POSTV_A(AD)                                          \
    switch (y_dtype) {                                       \
        case TCQ_F32: POSTV_Y(AD, TCQ_F32); break;           \
        case TCQ_BF16: POSTV_Y(AD, TCQ_BF16); break;         \
        case TCQ_F16: POSTV_Y(AD, TCQ_F16); break;           \
        default: return TCQ_ERR_DTYPE;                       \
    }
    switch (acc_dtype) {
        case TCQ_I32: POSTV_A(TCQ_I32); break;
        case TCQ_F32: POSTV_A(TCQ_F32); break;
        case TCQ_BF16: POSTV_A(TCQ_BF16); break;
        default: return TCQ_ERR_DTYPE;
    }
    return launch_status();
}

// Up to three layers whose accumulator columns, row scales, signs and biases lie side by side (layer i from column
// n0 + ... + n(i-1)); a layer with n <= 0 ends the list. BF16 outputs, the first optionally through the GELU table.
static int post_side_by_side(const void* acc, int acc_dtype, const float* s, const float* rs, const int8_t* sv, const float* bias,
                             const uint16_t* gelu_lut, void* y0, void* y1, void* y2, int M, int n0, int n1, int n2, int lda,
                             int gelu0, tcq_stream_t stream) {
    const int n[3] = {n0, n1, n2};
    void* ys[3] = {y0, y1, y2};
    tcq_post_seg segs[3];
    int nseg = 0, col = 0;
    for (int i = 0; i < 3 && n[i] > 0; ++i) {
        if (!ys[i]) return TCQ_ERR_ARG;
        segs[nseg++] = tcq_post_seg{acc, rs ? rs + col : nullptr, sv ? sv + col : nullptr, bias ? bias + col : nullptr, ys[i], lda, col, n[i],
                                    gelu0 && i == 0};
        col += n[i];
    }
    if (nseg == 0) return TCQ_ERR_ARG;
    return tcq_post_group(segs, nseg, acc_dtype, s, gelu_lut, TCQ_BF16, M, stream);
}

extern "C" int tcq_post3(const void* acc, int acc_dtype, const float* s, const float* rs, const int8_t* sv, const float* bias, void* y0,
                         void* y1, void* y2, int M, int n0, int n1, int n2, int lda, tcq_stream_t stream) {
    if (n0 <= 0 || n1 <= 0 || n2 <= 0) return TCQ_ERR_ARG;
    return post_side_by_side(acc, acc_dtype, s, rs, sv, bias, nullptr, y0, y1, y2, M, n0, n1, n2, lda, 0, stream);
}

extern "C" int tcq_postg3(const void* acc, int acc_dtype, const float* s, const float* rs, const int8_t* sv, const float* bias,
                          const uint16_t* gelu_lut, void* y0, void* y1, void* y2, int M, int n0, int n1, int n2, int lda, int gelu0,
                          tcq_stream_t stream) {
    if (n0 <= 0 || n1 <= 0) return TCQ_ERR_ARG;
    return post_side_by_side(acc, acc_dtype, s, rs, sv, bias, gelu_lut, y0, y1, y2, M, n0, n1, n2 > 0 ? n2 : 0, lda, gelu0, stream);
}

static size_t norm_lds(int K) { return row_lds(K) + (size_t)(K / 16) * sizeof(float); }

extern "C" int tcq_rmsnorm(const void* x, const void* w, float eps, void* y, int M, int K, tcq_stream_t stream) {
    if (!x || !w || !y || M <= 0 || K <= 0) return TCQ_ERR_ARG;
    if (K % 16 || K > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    const int vec = al16(x) && al16(y) && al16(w);
    launch_k(k_rmsnorm, dim3(M), dim3(row_threads(M, K)), norm_lds(K), (hipStream_t)stream, (const u16*)x, (const u16*)w, eps,
             (u16*)y, K, vec);
    return launch_status();
}

extern "C" int tcq_norm_pre(const void* x, const void* w, float eps, const int8_t* su, int8_t* q, int32_t* q4, int ldq, float* scale,
                            int M, int K, tcq_stream_t stream) {
    if (!x || !w || !su || !scale || (!q && !q4) || M <= 0 || K <= 0 || q4_bad(q4, ldq, M)) return TCQ_ERR_ARG;
    if (K % 16 || K > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    if (q4_tb_shape_bad(q4, ldq, K)) return TCQ_ERR_SHAPE;
    if (q4 && ldq == TCQ_LDQ_TOKEN_BLOCKS && !al16(q4)) return TCQ_ERR_ALIGN;
    const int vec = al16(x) && al16(w) && al16(su);
    launch_k(k_norm_pre, dim3(M), dim3(row_threads(M, K)), norm_lds(K), (hipStream_t)stream, (const u16*)x, (const u16*)w, eps,
             (const i8*)su, (i8*)q, (int*)q4, ldq, scale, K, vec);
    return launch_status();
}

extern "C" int tcq_post_add_norm_pre(const void* acc, int acc_dtype, int lda, int col0, const float* s, const float* rs,
                                     const int8_t* sv, const float* bias, const void* x, void* xout, const void* w, float eps,
                                     const int8_t* su, int8_t* q, int32_t* q4, int ldq, float* scale, int M, int N,
                                     tcq_stream_t stream) {
    if ((acc_dtype & TCQ_K_PARTS2) && (acc_dtype & TCQ_K_PARTS4)) return TCQ_ERR_ARG;
    const int parts = (acc_dtype & TCQ_K_PARTS4) ? 4 : (acc_dtype & TCQ_K_PARTS2) ? 2 : 1;
    acc_dtype &= ~(TCQ_K_PARTS2 | TCQ_K_PARTS4);
    if (parts > 1 && acc_dtype != TCQ_I32) return TCQ_ERR_DTYPE;
    if (parts > 1 && (size_t)parts * M * lda >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
    if (!acc || !sv || !x || !xout || M <= 0 || N <= 0 || col0 < 0 || lda < col0 + N) return TCQ_ERR_ARG;
    if ((acc_dtype == TCQ_I32 && (!s || !rs)) || (acc_dtype == TCQ_BF16 && !rs)) return TCQ_ERR_ARG;
    if (w && (!su || !scale || (!q && !q4) || q4_bad(q4, ldq, M))) return TCQ_ERR_ARG;
    if (N % 16 || N > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    if (q4_tb_shape_bad(q4, ldq, N)) return TCQ_ERR_SHAPE;
    if (q4 && ldq == TCQ_LDQ_TOKEN_BLOCKS && !al16(q4)) return TCQ_ERR_ALIGN;
    const int asz = dsize(acc_dtype);
    const int vec = al16(acc) && ((size_t)lda * asz) % 16 == 0 && ((size_t)col0 * asz) % 16 == 0 && (!rs || al16(rs));
    const int svec = al16(sv) && al16(x) && al16(xout) && (!bias || al16(bias)) && (!w || (al16(w) && al16(su)));
    hipStream_t st = (hipStream_t)stream;
    const u16 *xp = (const u16*)x, *wp = (const u16*)w;
    // register + transpose engine, 16 values per thread: power-of-two rows of 1024 .. 4096, aligned (measured on MI355X
    // against the register path: 50 x 1024 5.4 us against 6.9, 1 x 2048 5.7 against 7.5, 800 x 4096 13.7 against 19.5; with
    // 32 values per thread 2048-wide rows of few tokens run slower than the register path)
    // few rows of 1024 / 2048 with the norm: the no-transpose engine, 4 values per thread on 4 / 8 waves
    if (M <= 64 && w && !bias && (N == 1024 || N == 2048) && vec && svec && (!q || al16(q))) {
#define PANV(AD, L, NWP) launch_k(k_post_add_norm_pre_wv<AD, L, NWP>, dim3(M), dim3(64 * NWP), 0, st, acc, lda, col0, s, rs,   \
                                  (const i8*)sv, xp, (u16*)xout, wp, eps, (const i8*)su, (i8*)q, (int*)q4, ldq, scale, parts)
#define PANVW(L, NWP)                                    \
    switch (acc_dtype) {                                 \
        case TCQ_I32: PANV(TCQ_I32, L, NWP); break;      \
        case TCQ_F32: PANV(TCQ_F32, L, NWP); break;      \
        case TCQ_BF16: PANV(TCQ_BF16, L, NWP); break;    \
        default: return TCQ_ERR_DTYPE;                   \
    }
        if (N == 1024) { PANVW(10, 4); } else { PANVW(11, 8); }
#undef PANVW
#undef PANV
        return launch_status();
    }
    if ((N == 1024 || N == 2048 || N == 4096) && vec && svec && (!q || al16(q))) {
        const size_t tsh = (size_t)(lds_words(N) + N / 16) * sizeof(float);
#define PANT(AD, L, LE) launch_k(k_post_add_norm_pre_tw<AD, L, LE>, dim3(M), dim3(1 << (L - LE)), tsh, st, acc, lda, col0, s, rs, \
                                 (const i8*)sv, bias, xp, (u16*)xout, wp, eps, (const i8*)su, (i8*)q, (int*)q4, ldq, scale, parts)
#define PANW(L, LE)                                      \
    switch (acc_dtype) {                                 \
        case TCQ_I32: PANT(TCQ_I32, L, LE); break;       \
        case TCQ_F32: PANT(TCQ_F32, L, LE); break;       \
        case TCQ_BF16: PANT(TCQ_BF16, L, LE); break;     \
        default: return TCQ_ERR_DTYPE;                   \
    }
        // few rows (latency): 8 values per thread, twice the threads per row (four register passes); many rows: 16
        const bool wide = M <= 64;
        switch (N) {
            case 1024: if (wide) { PANW(10, 3); } else { PANW(10, 4); } break;
            case 2048: if (wide) { PANW(11, 3); } else { PANW(11, 4); } break;
            default: if (wide) { PANW(12, 3); } else { PANW(12, 4); } break;
        }
#undef PANW
#undef PANT
        return launch_status();
    }
    // register path: power-of-two rows of 1024 .. 16384 (one 16-element chunk per thread, at least one full wave), aligned
    if ((N & (N - 1)) == 0 && N >= 1024 && vec && svec && (!q || al16(q))) {
#define PANR(AD) launch_k(k_post_add_norm_pre_reg<AD>, dim3(M), dim3(N / 16), (size_t)N * sizeof(float), st, acc, lda, col0, s, rs, \
                          (const i8*)sv, bias, xp, (u16*)xout, wp, eps, (const i8*)su, (i8*)q, (int*)q4, ldq, scale, N, parts)
        switch (acc_dtype) {
            case TCQ_I32: PANR(TCQ_I32); break;
            case TCQ_F32: PANR(TCQ_F32); break;
            case TCQ_BF16: PANR(TCQ_BF16); break;
            default: return TCQ_ERR_DTYPE;
        }
#undef PANR
        return launch_status();
    }
    if (parts > 1) return TCQ_ERR_UNSUPPORTED;         // K parts: register paths only
    // 512 threads at most: the side vectors the kernel loads ahead need more than the 128 registers of 1024-thread groups
    const dim3 grid(M), block(row_threads(M, N) < 512 ? row_threads(M, N) : 512);
    const size_t sh = norm_lds(N);
#define PANP(AD) launch_k(k_post_add_norm_pre<AD>, grid, block, sh, st, acc, lda, col0, s, rs, (const i8*)sv, bias, xp, (u16*)xout, \
                          wp, eps, (const i8*)su, (i8*)q, (int*)q4, ldq, scale, N, vec, svec)
    switch (acc_dtype) {
        case TCQ_I32: PANP(TCQ_I32); break;
        case TCQ_F32: PANP(TCQ_F32); break;
        case TCQ_BF16: PANP(TCQ_BF16); break;
        default: return TCQ_ERR_DTYPE;
    }
    return launch_status();
}
