// Row helpers shared by the row kernels (tcq_walsh.hip) and the products that run a row kernel as their prologue
// (tcq_gemm_small.hip): 16-element chunk loads / stores, the fixed-order sum of squares, accumulator chunks.
#pragma once
#include "tcq_device.h"

// ------------------------------------------------------------------------------------------------ 16-element chunks
// The row kernels keep every global access out of the Walsh passes: the passes read and write LDS only, and the
// side vectors (signs, bias, residual, norm weight) are read per 16-element chunk with 16-byte loads (vec) or element by
// element (rows whose base or length breaks the alignment), all loads of a chunk issued before any of them is used.
__device__ __forceinline__ void c16_bf16(const u16* p, bool vec, float (&v)[16]) {
    if (vec) {
        const uint4_t a = gptr((const uint4_t*)p)[0], b = gptr((const uint4_t*)p)[1];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[2 * k] = bf16_to_f32((u16)(a[k] & 0xffffu)); v[2 * k + 1] = bf16_to_f32((u16)(a[k] >> 16));
            v[8 + 2 * k] = bf16_to_f32((u16)(b[k] & 0xffffu)); v[9 + 2 * k] = bf16_to_f32((u16)(b[k] >> 16));
        }
    } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = bf16_to_f32(gptr(p)[k]);
    }
}
__device__ __forceinline__ void c16_store_bf16(u16* p, bool vec, const u16 (&h)[16]) {
    if (vec) {
        uint4_t a, b;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            a[k] = (u32)h[2 * k] | ((u32)h[2 * k + 1] << 16);
            b[k] = (u32)h[8 + 2 * k] | ((u32)h[9 + 2 * k] << 16);
        }
        gptr((uint4_t*)p)[0] = a;
        gptr((uint4_t*)p)[1] = b;
    } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) gptr(p)[k] = h[k];
    }
}
__device__ __forceinline__ void c16_i8(const i8* p, bool vec, float (&v)[16]) {
    if (vec) {
        const uint4_t a = gptr((const uint4_t*)p)[0];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = (float)(i8)(a[k >> 2] >> (8 * (k & 3)));
    } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = (float)gptr(p)[k];
    }
}
__device__ __forceinline__ void c16_f32(const float* p, bool vec, float (&v)[16]) {
    if (vec) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint4_t a = gptr((const uint4_t*)p)[q];
#pragma unroll
            for (int k = 0; k < 4; ++k) v[4 * q + k] = __uint_as_float(a[k]);
        }
    } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = gptr(p)[k];
    }
}

// Sum of squares of a row in an order fixed by K alone: chunk sums of 16 consecutive values (sequential, part[j] for chunk
// j), then a pairwise tree over the chunks, stage h adding chunk j + h into chunk j for j a multiple of 2h. Stages h < 64 run
// in registers across the lanes of a wave (chunks past the end count as +0, which leaves every partial sum unchanged), the
// rest over the per-wave results. part: the K / 16 chunk sums (LDS, complete on entry: the caller synchronises); red: >= 16
// floats of LDS. Every thread gets the total. Ends with a barrier.
__device__ __forceinline__ float chunk_sumsq(const float (&v)[16]) {
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) a = a + v[k] * v[k];
    return a;
}
__device__ __forceinline__ float tree_total(const float* part, float* red, int K) {
    const int C = K >> 4, groups = (C + 63) >> 6;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int g = wid; g < groups; g += nw) {
        const int j = (g << 6) + lane;
        float v = j < C ? part[j] : 0.f;
        // pairwise tree over the 64 lanes (stride 1, 2, 4, 8 inside the rows, then 16 and 32): lane l adds lane l + h for l
        // a multiple of 2h; the other lanes compute values no kept lane reads
        v = v + dpp<0x101>(v);
        v = v + dpp<0x102>(v);
        v = v + dpp<0x104>(v);
        v = v + dpp<0x108>(v);
        v = (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
        if (lane == 0) red[g] = v;
    }
    __syncthreads();
    float r[16];
#pragma unroll
    for (int g = 0; g < 16; ++g) r[g] = g < groups ? red[g] : 0.f;
#pragma unroll
    for (int h = 1; h < 16; h <<= 1)
#pragma unroll
        for (int g = 0; g + h < 16; g += 2 * h) r[g] = r[g] + r[g + h];
    __syncthreads();
    return r[0];
}

// Accumulator chunk 16 t .. 16 t + 15 of a row (scaled as tcq_post scales it: int32 * s * rs, BF16 * rs, FP32 as is), loaded at kernel entry. int32 K parts (parts > 1,
// part p at acc + p * pstride) are added in int32 first: the same sum as one part.
template <int ADT>
__device__ __forceinline__ void acc_chunk(const void* acc, size_t base, float st, const float* rs, float (&v)[16], int parts = 1,
                                          size_t pstride = 0) {
    if (ADT == TCQ_BF16) {
        const Raw16<2> a = raw16<2>((const u16*)acc + base, true);
        const Raw16<4> r4 = raw16<4>(rs, true);
        float r[16];
        cv16(a, v);
        cv16(r4, r);
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = v[k] * r[k];
    } else {
        Raw16<4> a = raw16<4>((const u32*)acc + base, true);
        if (ADT == TCQ_I32) {
            Raw16<4> ap[3];
#pragma unroll
            for (int p = 1; p < 4; ++p)
                if (p < parts) ap[p - 1] = raw16<4>((const u32*)acc + base + p * pstride, true);
            const Raw16<4> r4 = raw16<4>(rs, true);
#pragma unroll
            for (int p = 1; p < 4; ++p)
                if (p < parts) {
#pragma unroll
                    for (int k = 0; k < 16; ++k) a.r[k >> 2][k & 3] = (u32)((int)a.r[k >> 2][k & 3] + (int)ap[p - 1].r[k >> 2][k & 3]);
                }
            float r[16];
            cv16(r4, r);
#pragma unroll
            for (int k = 0; k < 16; ++k) v[k] = ((float)(int)a.r[k >> 2][k & 3] * st) * r[k];
        } else {
            cv16(a, v);
        }
    }
}

// ------------------------------------------------------------------------------------ epilogue + residual + norm of a row
// Arguments of tcq_post_add_norm_pre for one launch (device copies of its pointers).
struct PanpArgs {
    const void* acc;
    const float* s;
    const float* rs;
    const i8* sv;
    const float* bias;
    const u16* x;
    u16* xout;
    const u16* w;
    const i8* su;
    int lda, col0, parts;
    size_t pstride;          // elements between K parts of acc
    float eps;
};

// tcq_post_add_norm_pre of token tok up to the rotate + quantize, on the register + transpose engine with 2^LE values per
// thread: a = bf16((walsh(acc) * c) * sv (+ bias)), xout = bf16(x + a) (stored when `store`), then, when w is given,
// v = bf16((xout * r) * (1 + w)) * su with r from the fixed-order sum of squares. v ends in natural layout (thread t holds
// values 2^LE t ..), ready for tw_rotate_quantize. Threads from 2^(L - LE) on hold no values; they load and store nothing
// but meet every barrier. xs: lds_words(2^L) floats, part: 2^L / 16 floats, red: 16 floats (LDS). Returns false (uniform)
// when there is no norm (w NULL): v then holds xout. mid() runs once every thread's accumulator loads have been consumed
// (a caller issues its own loads there, when the accumulator registers are free again).
struct NoMid {
    __device__ void operator()() const {}
};
// BIAS = false: A.bias is ignored (callers that have none save its registers).
// 8-element pieces (the eight-values-per-thread engine): loads of 8 consecutive values as FP32.
__device__ __forceinline__ void ld8_i8v(const i8* p, float (&v)[8]) {
    const u64 w = *gptr((const u64*)p);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = (float)(i8)(w >> (8 * k));
}
__device__ __forceinline__ void ld8_bf16v(const u16* p, float (&v)[8]) {
    const uint4_t a = gptr((const uint4_t*)p)[0];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        v[2 * k] = __uint_as_float(a[k] << 16);
        v[2 * k + 1] = __uint_as_float(a[k] & 0xffff0000u);
    }
}
__device__ __forceinline__ void ld8_f32v(const float* p, float (&v)[8]) {
    const uint4_t a = gptr((const uint4_t*)p)[0], b = gptr((const uint4_t*)p)[1];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        v[k] = __uint_as_float(a[k]);
        v[4 + k] = __uint_as_float(b[k]);
    }
}
// acc_chunk for 8 values
template <int ADT>
__device__ __forceinline__ void acc_piece8(const void* acc, size_t base, float st, const float* rs, float (&v)[8], int parts,
                                           size_t pstride) {
    if (ADT == TCQ_BF16) {
        float r[8];
        ld8_bf16v((const u16*)acc + base, v);
        ld8_f32v(rs, r);
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = v[k] * r[k];
    } else if (ADT == TCQ_I32) {
        uint4_t a[2], ap[3][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) a[h] = gptr((const uint4_t*)((const u32*)acc + base))[h];
#pragma unroll
        for (int p = 1; p < 4; ++p)
            if (p < parts) {
#pragma unroll
                for (int h = 0; h < 2; ++h) ap[p - 1][h] = gptr((const uint4_t*)((const u32*)acc + base + p * pstride))[h];
            }
        float r[8];
        ld8_f32v(rs, r);
#pragma unroll
        for (int p = 1; p < 4; ++p)
            if (p < parts) {
#pragma unroll
                for (int k = 0; k < 8; ++k) a[k >> 2][k & 3] = (u32)((int)a[k >> 2][k & 3] + (int)ap[p - 1][k >> 2][k & 3]);
            }
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = ((float)(int)a[k >> 2][k & 3] * st) * r[k];
    } else {
        ld8_f32v((const float*)acc + base, v);
    }
}

// panp_tw with 8 values per thread (rows of 2^L on 2^(L - 3) threads): the same operations in the same order. The sum of
// squares keeps its 16-element chunks: the even thread of a pair sums its 8 squares from 0, the odd one continues from the
// even one's partial sum (a DPP move from the lane below), so every chunk sum is the sequential one.
template <int ADT, int L, bool BIAS, class F>
__device__ __forceinline__ bool panp_tw8(const PanpArgs& A, int tok, bool store, float (&v)[8], float* xs, float* part,
                                         float* red, F&& mid) {
    constexpr int N = 1 << L;
    const int t = threadIdx.x, i0 = 8 * t;
    const bool on = t < (N >> 3);                                      // whole waves (N >= 512)
    const size_t row = (size_t)tok * N, base = (size_t)tok * A.lda + A.col0 + i0;
    float sg[8], xv[8], b[8], wv[8], sn[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = 0.f;
    if (on) {
        ld8_i8v(A.sv + i0, sg);
        ld8_bf16v(A.x + row + i0, xv);
        if (BIAS && A.bias) ld8_f32v(A.bias + i0, b);
        if (A.w) {
            ld8_bf16v(A.w + i0, wv);
            ld8_i8v(A.su + i0, sn);
        }
        acc_piece8<ADT>(A.acc, base, ADT == TCQ_I32 ? A.s[tok] : 1.f, A.rs ? A.rs + i0 : nullptr, v, A.parts, A.pstride);
    }
    mid();
    const float c = (float)(1.0 / __builtin_sqrt((double)N));
    tw_walsh<L, 3>(v, xs);
    tw_to_natural<L, 3>(v, xs);
    if (on) {
        float a[8];
        u16 xn[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            a[k] = (v[k] * c) * sg[k];
            if (BIAS && A.bias) a[k] = a[k] + b[k];
        }
        bf16_round<4>(a, xn);                                          // a = bf16(post output)
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = xv[k] + a[k];
        bf16_round<4>(v, xn);                                          // xout = bf16(x + a)
        if (store)
            *gptr((uint4_t*)(A.xout + row + i0)) = uint4_t{(u32)xn[0] | ((u32)xn[1] << 16), (u32)xn[2] | ((u32)xn[3] << 16),
                                                           (u32)xn[4] | ((u32)xn[5] << 16), (u32)xn[6] | ((u32)xn[7] << 16)};
        if (A.w) {
            float s0 = 0.f;
#pragma unroll
            for (int k = 0; k < 8; ++k) s0 = s0 + v[k] * v[k];
            float s1 = dpp<0x111>(s0);                                 // row_shr:1: the even lane's partial sum
#pragma unroll
            for (int k = 0; k < 8; ++k) s1 = s1 + v[k] * v[k];
            if (t & 1) part[t >> 1] = s1;
        }
    }
    if (!A.w) return false;                                             // uniform
    __syncthreads();
    const float ss = tree_total(part, red, N);
    const float r = 1.f / __builtin_sqrtf(ss / (float)N + A.eps);
    if (on) {
        float nv[8];
        u16 nh[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) nv[k] = (v[k] * r) * (1.f + wv[k]);
        bf16_round<4>(nv, nh);
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = nv[k] * sn[k];
    }
    return true;
}

template <int ADT, int L, int LE, bool BIAS, class F>
__device__ __forceinline__ bool panp_tw16(const PanpArgs& A, int tok, bool store, float (&v)[1 << LE], float* xs, float* part,
                                          float* red, F&& mid) {
    constexpr int N = 1 << L, E = 1 << LE, NP = E / 16;
    const int t = threadIdx.x, i0 = E * t;
    const bool on = t < (N >> LE);
    const size_t row = (size_t)tok * N, base = (size_t)tok * A.lda + A.col0 + i0;
    Raw16<1> sv0[NP], su0[NP];
    Raw16<2> x0[NP], w0[NP];
    Raw16<4> b0[NP];
#pragma unroll
    for (int h = 0; h < NP; ++h) {
#pragma unroll
        for (int k = 0; k < 16; ++k) v[16 * h + k] = 0.f;
        if (on) {
            sv0[h] = raw16<1>(A.sv + i0 + 16 * h, true);
            x0[h] = raw16<2>(A.x + row + i0 + 16 * h, true);
            if (BIAS && A.bias) b0[h] = raw16<4>(A.bias + i0 + 16 * h, true);
            if (A.w) {
                w0[h] = raw16<2>(A.w + i0 + 16 * h, true);
                su0[h] = raw16<1>(A.su + i0 + 16 * h, true);
            }
        }
    }
    if (on) {
#pragma unroll
        for (int h = 0; h < NP; ++h)
            acc_chunk<ADT>(A.acc, base + 16 * h, ADT == TCQ_I32 ? A.s[tok] : 1.f, A.rs ? A.rs + i0 + 16 * h : nullptr, part16(v, h),
                           A.parts, A.pstride);
    }
    mid();
    const float c = (float)(1.0 / __builtin_sqrt((double)N));
    tw_walsh<L, LE>(v, xs);
    tw_to_natural<L, LE>(v, xs);
    if (on) {
#pragma unroll
        for (int h = 0; h < NP; ++h) {
            float sg[16], b[16], xv[16], a[16];
            u16 xn[16];
            cv16(sv0[h], sg);
            if (BIAS && A.bias) cv16(b0[h], b);
            cv16(x0[h], xv);
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                a[k] = (v[16 * h + k] * c) * sg[k];
                if (BIAS && A.bias) a[k] = a[k] + b[k];
            }
            bf16_round<8>(a, xn);                                      // a = bf16(post output)
#pragma unroll
            for (int k = 0; k < 16; ++k) v[16 * h + k] = xv[k] + a[k];
            bf16_round<8>(&v[16 * h], xn);                             // xout = bf16(x + a)
            if (store) c16_store_bf16(A.xout + row + i0 + 16 * h, true, xn);
            if (A.w) part[NP * t + h] = chunk_sumsq(part16(v, h));
        }
    }
    if (!A.w) return false;                                             // uniform
    __syncthreads();
    const float ss = tree_total(part, red, N);
    const float r = 1.f / __builtin_sqrtf(ss / (float)N + A.eps);
    if (on) {
#pragma unroll
        for (int h = 0; h < NP; ++h) {
            float wv[16], sn[16];
            cv16(w0[h], wv);
            cv16(su0[h], sn);
            float nv[16];
            u16 nh[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) nv[k] = (v[16 * h + k] * r) * (1.f + wv[k]);
            bf16_round<8>(nv, nh);
#pragma unroll
            for (int k = 0; k < 16; ++k) v[16 * h + k] = nv[k] * sn[k];
        }
    }
    return true;
}

template <int ADT, int L, int LE, bool BIAS = true, class F = NoMid>
__device__ __forceinline__ bool panp_tw(const PanpArgs& A, int tok, bool store, float (&v)[1 << LE], float* xs, float* part,
                                        float* red, F&& mid = NoMid{}) {
    if constexpr (LE == 3) return panp_tw8<ADT, L, BIAS>(A, tok, store, v, xs, part, red, mid);
    else return panp_tw16<ADT, L, LE, BIAS>(A, tok, store, v, xs, part, red, mid);
}

// --------------------------------------------------------- rows of 1024 / 2048 on four or eight waves, no transposes
// LDS of panp_waves / waves_rotate_quantize: the exchange rows of wave_walsh, the per-wave sums and maxima. The two take
// WAVES_SYNCS calls of sync() together (two each).
template <int N>
struct WavesLdsN {
    float xs[N];
    float red[16];
};
typedef WavesLdsN<2048> WavesLds;
constexpr int WAVES_SYNCS = 4;

// panp_tw for token tok of a 2^L-wide row (L = 10 or 11) with the norm (A.w set, no bias) on waves 0 .. NWP - 1 (NWP = 4
// or 8: E = 2^L / 64 / NWP = 4 or 8 values per thread), with two sync() points (barriers that a caller's other waves may
// meet while they do other work): the Walsh on wave_walsh; the chunk sums of squares in order, each chunk's 16 values
// over 16 / E consecutive lanes (each lane continues the sum of the lane below, a DPP move), so the last lane of the
// group holds the sequential sum; their pairwise tree over the lanes of a wave by DPP inside the 16-lane rows, then
// across the rows, and over the waves through LDS. The tree is tree_total's (chunk j + h into chunk j at level h), so
// every value equals panp_tw's bit for bit. Threads of waves < NWP call it; v ends in natural layout for
// waves_rotate_quantize. mid() runs once the accumulator loads have been consumed. xout is stored when `store`.
template <int ADT, int NWP, int L = 11, class F, class SY>
__device__ __forceinline__ void panp_waves(const PanpArgs& A, int tok, bool store, float (&v)[(1 << L) / 64 / NWP], WavesLds& Q,
                                           F&& mid, SY&& sync) {
    constexpr int N = 1 << L, E = N / 64 / NWP, LE = E == 8 ? 3 : 2, LPC = 16 / E;
    static_assert((L == 10 || L == 11) && (E == 4 || E == 8), "rows of 1024 or 2048, 4 or 8 values per thread");
    const int t = threadIdx.x, i0 = E * t, lane = t & 63, w = t >> 6;
    const size_t row = (size_t)tok * N, base = (size_t)tok * A.lda + A.col0 + i0;
    float sg[E], xv[E], wv[E], sn[E];
    auto ld_i8 = [&](const i8* p, float (&o)[E]) {
        if constexpr (E == 8) {
            ld8_i8v(p, o);
        } else {
            const u32 x = *gptr((const u32*)p);
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = (float)(i8)(x >> (8 * k));
        }
    };
    auto ld_bf16 = [&](const u16* p, float (&o)[E]) {
        if constexpr (E == 8) {
            ld8_bf16v(p, o);
        } else {
            const uint2_t x = *gptr((const uint2_t*)p);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                o[2 * k] = __uint_as_float(x[k] << 16);
                o[2 * k + 1] = __uint_as_float(x[k] & 0xffff0000u);
            }
        }
    };
    ld_i8(A.sv + i0, sg);
    ld_bf16(A.x + row + i0, xv);
    ld_bf16(A.w + i0, wv);
    ld_i8(A.su + i0, sn);
    const float st = ADT == TCQ_I32 ? A.s[tok] : 1.f;
    if constexpr (E == 8) {
        acc_piece8<ADT>(A.acc, base, st, A.rs ? A.rs + i0 : nullptr, v, A.parts, A.pstride);
    } else if constexpr (ADT == TCQ_I32) {
        uint4_t a = *gptr((const uint4_t*)((const u32*)A.acc + base));
        uint4_t ap[3];
#pragma unroll
        for (int p = 1; p < 4; ++p)
            if (p < A.parts) ap[p - 1] = *gptr((const uint4_t*)((const u32*)A.acc + base + p * A.pstride));
        const float4_t r = *gptr((const float4_t*)(A.rs + i0));
#pragma unroll
        for (int p = 1; p < 4; ++p)
            if (p < A.parts) {
#pragma unroll
                for (int k = 0; k < 4; ++k) a[k] = (u32)((int)a[k] + (int)ap[p - 1][k]);
            }
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = ((float)(int)a[k] * st) * r[k];
    } else if constexpr (ADT == TCQ_BF16) {
        ld_bf16((const u16*)A.acc + base, v);
        const float4_t r = *gptr((const float4_t*)(A.rs + i0));
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = v[k] * r[k];
    } else {
        const float4_t a = *gptr((const float4_t*)((const float*)A.acc + base));
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = a[k];
    }
    mid();
    const float c = (float)(1.0 / __builtin_sqrt((double)N));
    wave_walsh<LE, NWP>(v, Q.xs, sync);
    float a[E];
    u16 xn[E];
#pragma unroll
    for (int k = 0; k < E; ++k) a[k] = (v[k] * c) * sg[k];
    bf16_round<E / 2>(a, xn);                                          // a = bf16(post output)
#pragma unroll
    for (int k = 0; k < E; ++k) v[k] = xv[k] + a[k];
    bf16_round<E / 2>(v, xn);                                          // xout = bf16(x + a)
    if (store) {
        u32 x2[E / 2];
#pragma unroll
        for (int k = 0; k < E / 2; ++k) x2[k] = (u32)xn[2 * k] | ((u32)xn[2 * k + 1] << 16);
        if constexpr (E == 8) *gptr((uint4_t*)(A.xout + row + i0)) = uint4_t{x2[0], x2[1], x2[2], x2[3]};
        else *gptr((uint2_t*)(A.xout + row + i0)) = uint2_t{x2[0], x2[1]};
    }
    // chunk sums: lane l continues lane l - 1's partial sum (row_shr:1), LPC lanes per chunk
    float cs = 0.f;
#pragma unroll
    for (int k = 0; k < E; ++k) cs = cs + v[k] * v[k];
#pragma unroll
    for (int g = 1; g < LPC; ++g) {
        float p = dpp<0x111>(cs);
#pragma unroll
        for (int k = 0; k < E; ++k) p = p + v[k] * v[k];
        cs = p;
    }
    // lane LPC j + LPC - 1 now holds chunk j of the wave; the tree inside the rows (row_shl by LPC, 2 LPC, .. 8)
#pragma unroll
    for (int h = LPC; h < 16; h *= 2) cs = cs + (h == 2 ? dpp<0x102>(cs) : h == 4 ? dpp<0x104>(cs) : dpp<0x108>(cs));
    const float ws = (lane_value(cs, LPC - 1) + lane_value(cs, 16 + LPC - 1)) +
                     (lane_value(cs, 32 + LPC - 1) + lane_value(cs, 48 + LPC - 1));
    if (lane == 0) Q.red[w] = ws;
    sync();
    // the waves' sums: levels 16 / 32 chunks (E = 4 / 8) and up, in tree_total's pairing for 2^L / 16 chunks
    float ss;
    if constexpr (NWP == 4) ss = (Q.red[0] + Q.red[1]) + (Q.red[2] + Q.red[3]);
    else ss = ((Q.red[0] + Q.red[1]) + (Q.red[2] + Q.red[3])) + ((Q.red[4] + Q.red[5]) + (Q.red[6] + Q.red[7]));
    const float r = 1.f / __builtin_sqrtf(ss / (float)N + A.eps);
    float nv[E];
    u16 nh[E];
#pragma unroll
    for (int k = 0; k < E; ++k) nv[k] = (v[k] * r) * (1.f + wv[k]);
    bf16_round<E / 2>(nv, nh);
#pragma unroll
    for (int k = 0; k < E; ++k) v[k] = nv[k] * sn[k];
}

// tw_rotate_quantize of a 2^L-wide row (token tok) on waves 0 .. NWP - 1 (v: E = 2^L / 64 / NWP values per thread, natural
// layout), with two sync() points: wave_walsh, the row maximum over the waves through LDS, the INT8 row into qs (LDS, E
// bytes per thread), q (row tok), q4 (the word layout, or token blocks when ldq is TCQ_LDQ_TOKEN_BLOCKS) as given; the
// scale into *scs and scale[tok] as given. The same values as tw_rotate_quantize<L, LE>.
template <int NWP, int L = 11, class QL, class SY>
__device__ __forceinline__ void waves_rotate_quantize(float (&v)[(1 << L) / 64 / NWP], QL& Q, u32* qs, float* scs, i8* q, float* scale,
                                                      SY&& sync, int tok = 0, int* q4 = nullptr, int ldq = 0) {
    constexpr int N = 1 << L, E = N / 64 / NWP, LE = E == 8 ? 3 : 2;
    static_assert((E == 4 || E == 8) && sizeof(Q.xs) >= N * sizeof(float), "4 or 8 values per thread, an exchange row of N");
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const float c = (float)(1.0 / __builtin_sqrt((double)N));
    wave_walsh<LE, NWP>(v, Q.xs, sync);
    float mx = 0.f;
#pragma unroll
    for (int k = 0; k < E; ++k) {
        v[k] = v[k] * c;
        mx = fmaxf(mx, fabsf(v[k]));
    }
    mx = wave_max(mx);
    if (lane == 0) Q.red[8 + w] = mx;
    sync();
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < NWP; ++i) m = fmaxf(m, Q.red[8 + i]);
    const float sc = token_scale(m);
    if (t == 0) {
        if (scs) *scs = sc;
        if (scale) scale[tok] = sc;
    }
    const QScale S = qscale(sc);
    u32 words[E / 4];
#pragma unroll
    for (int k4 = 0; k4 < E / 4; ++k4)
        words[k4] = (u32)(q8(v[4 * k4], S) & 0xff) | ((u32)(q8(v[4 * k4 + 1], S) & 0xff) << 8) |
                    ((u32)(q8(v[4 * k4 + 2], S) & 0xff) << 16) | ((u32)(q8(v[4 * k4 + 3], S) & 0xff) << 24);
    const bool tb = q4 && ldq == TCQ_LDQ_TOKEN_BLOCKS;
    if constexpr (E == 8) {
        const u64 d = (u64)words[0] | ((u64)words[1] << 32);
        if (qs) *(u64*)(qs + 2 * t) = d;
        if (q) *gptr((u64*)(q + (size_t)tok * N + 8 * t)) = d;
        if (tb) *gptr((u64*)((i8*)q4 + tb_offset(tok, 8 * t, N))) = d;
    } else {
        if (qs) qs[t] = words[0];
        if (q) *gptr((u32*)(q + (size_t)tok * N + 4 * t)) = words[0];
        if (tb) *gptr((u32*)((i8*)q4 + tb_offset(tok, 4 * t, N))) = words[0];
    }
    if (q4 && !tb) {
#pragma unroll
        for (int k4 = 0; k4 < E / 4; ++k4) q4[(size_t)((E / 4) * t + k4) * ldq + tok] = (int)words[k4];
    }
}

// The rotate + quantize input of a BF16 row (tcq_pre's first steps): thread t's 2^LE contiguous values x[2^LE t ..] * su,
// as FP32 in v (natural layout, ready for tw_rotate_quantize). Threads from 2^(L - LE) on hold no values (zeros). mid()
// runs once the loaded words have been consumed.
template <int L, int LE, class F = NoMid>
__device__ __forceinline__ void pre_row_tw(const u16* x, const i8* su, float (&v)[1 << LE], F&& mid = NoMid{}) {
    constexpr int E = 1 << LE;
    const int t = threadIdx.x, i0 = E * t;
    const bool on = t < (1 << (L - LE));
    Raw16<1> s0[E / 16];
    uint4_t raw[E / 8];
    if (on) {
#pragma unroll
        for (int h = 0; h < E / 16; ++h) s0[h] = raw16<1>(su + i0 + 16 * h, true);
#pragma unroll
        for (int j = 0; j < E / 8; ++j) raw[j] = gptr((const uint4_t*)(x + i0))[j];
    }
#pragma unroll
    for (int k = 0; k < E; ++k) v[k] = on ? bf16_to_f32((u16)(raw[k >> 3][(k & 7) >> 1] >> (16 * (k & 1)))) : 0.f;
    if (on) {
#pragma unroll
        for (int h = 0; h < E / 16; ++h) {
            float sg[16];
            cv16(s0[h], sg);
#pragma unroll
            for (int k = 0; k < 16; ++k) v[16 * h + k] = v[16 * h + k] * sg[k];
        }
    }
    mid();
}
