// Device helpers shared by the TCQ kernels (gfx950, wave64).
//
// Number formats follow the reference arithmetic of deploy/tcq_kernels/tcq_format.py: BF16 round-to-nearest-even with the
// canonical NaN 0x7fc0 (c10::BFloat16; reference kernels.py:19-25), FP16 round-to-nearest-even (_Float16 conversion),
// IEEE FP32 division, round-half-even (v_rndne_f32). Every translation unit is built with -ffp-contract=off so that no
// a * b + c is contracted into an FMA (the reference compiles with --fmad=false, cuda_rt.py:53).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tcq_api.h"

typedef uint16_t u16;
typedef uint32_t u32;
typedef uint64_t u64;
typedef int8_t i8;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef int int4_t __attribute__((ext_vector_type(4)));
typedef u32 uint4_t __attribute__((ext_vector_type(4)));
typedef u32 uint2_t __attribute__((ext_vector_type(2)));
typedef u16 u16x2_t __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------------------------------------------------ conversions
__device__ __forceinline__ float bf16_to_f32(u16 b) { return __uint_as_float(((u32)b) << 16); }
// FP32 -> BF16, round to nearest even, every NaN -> 0x7fc0 (reference kernels.py:20-25). gfx950's v_cvt_pk_bf16_f32
// rounds to nearest even (subnormals kept: the kernels run with FP32 denormals on); only its NaN results differ (it keeps
// the sign and payload), so NaN inputs are replaced after the conversion.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u16 f32_to_bf16(float f) {
    const u16 h = __builtin_bit_cast(u16, (__bf16)f);
    return __builtin_isnan(f) ? (u16)0x7fc0 : h;
}
__device__ __forceinline__ u32 bf16_cvt2(float a, float b) {
    return __builtin_bit_cast(u32, __builtin_convertvector(float2_t{a, b}, bf16x2_t));
}
// the word of a converted pair with the half of each NaN input replaced by 0x7fc0 (one bitfield insert)
__device__ __forceinline__ u32 bf16_nan_fix(u32 w, float a, float b) {
    const u32 m = (__builtin_isnan(a) ? 0xffffu : 0u) | (__builtin_isnan(b) ? 0xffff0000u : 0u);
    return (m & 0x7fc07fc0u) | (~m & w);
}
// two values -> one word of two BF16 (a in the low half)
__device__ __forceinline__ u32 bf16x2(float a, float b) { return bf16_nan_fix(bf16_cvt2(a, b), a, b); }
// 2 NP values -> NP words (value 2p in the low half of word p): one conversion per pair; one unordered compare per pair
// into a wave-wide lane mask (scalar ORs) decides whether any lane of the wave holds a NaN, and only then does the wave run
// the fix-up (a uniform branch).
template <int NP>
__device__ __forceinline__ void bf16_pack(const float* v, u32* w) {
    u64 nan = 0;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        w[p] = bf16_cvt2(v[2 * p], v[2 * p + 1]);
        nan |= __builtin_amdgcn_ballot_w64(__builtin_isunordered(v[2 * p], v[2 * p + 1]));
    }
    if (__builtin_expect(nan != 0, false)) {
#pragma unroll
        for (int p = 0; p < NP; ++p) w[p] = bf16_nan_fix(w[p], v[2 * p], v[2 * p + 1]);
    }
}
// 2 NP values rounded to BF16 in place (each replaced by its BF16 value as FP32), the BF16 halves in h
template <int NP>
__device__ __forceinline__ void bf16_round(float* v, u16* h) {
    u32 w[NP];
    bf16_pack<NP>(v, w);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        h[2 * p] = (u16)(w[p] & 0xffffu);
        h[2 * p + 1] = (u16)(w[p] >> 16);
        v[2 * p] = __uint_as_float(w[p] << 16);
        v[2 * p + 1] = __uint_as_float(w[p] & 0xffff0000u);
    }
}
__device__ __forceinline__ float f16_to_f32(u16 h) { return (float)__builtin_bit_cast(_Float16, h); }
// FP32 -> FP16 of an FP32 value. The value is pinned in a register first: otherwise the compiler may fuse a preceding multiply
// and this conversion into one mixed-precision FMA (v_fma_mixlo_f16), a single rounding of the exact product, where the
// defined result rounds to FP32 and then to FP16 (the two differ when the FP32 product is an exact FP16 tie).
__device__ __forceinline__ u16 f32_to_f16(float f) {
    asm("" : "+v"(f));
    return __builtin_bit_cast(u16, (_Float16)f);
}

// load element i of a row of dtype `dt` as FP32 (exact for every supported input type)
__device__ __forceinline__ float load_as_f32(const void* p, size_t i, int dt) {
    switch (dt) {
        case TCQ_F32: return ((const float*)p)[i];
        case TCQ_BF16: return bf16_to_f32(((const u16*)p)[i]);
        case TCQ_F16: return f16_to_f32(((const u16*)p)[i]);
        case TCQ_I32: return (float)((const int*)p)[i];
        default: return 0.f;
    }
}
__device__ __forceinline__ void store_from_f32(void* p, size_t i, float v, int dt) {
    switch (dt) {
        case TCQ_F32: ((float*)p)[i] = v; break;
        case TCQ_BF16: ((u16*)p)[i] = f32_to_bf16(v); break;
        case TCQ_F16: ((u16*)p)[i] = f32_to_f16(v); break;
        default: break;
    }
}

// ------------------------------------------------------------------------------------------------- wave / block reductions
// Cross-lane moves inside 16-lane rows by DPP (a modifier of the consuming instruction, no trip through the LDS crossbar):
// dpp<C>(v) returns, in lane i, v of lane: quad_perm 0xB1 -> i ^ 1, 0x4E -> i ^ 2; row_ror:N (0x120 + N) -> row lane
// (i - N) mod 16; row_shl:N (0x100 + N) -> i + N within the row (0 past the row's end). Checked on MI355X lane by lane.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float lane_value(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }

// max over the 16 lanes of each row, in every lane of the row (max is exact in any order)
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x124>(v));
    return fmaxf(v, dpp<0x128>(v));
}
// sum over the 16 lanes of each row, the same bits in every lane of the row: each step adds the partial sum of a disjoint
// class of lanes (shifts 8, 4, 2, 1), and the two lanes of every pair add the same two values
__device__ __forceinline__ float row16_sum(float v) {
    v = v + dpp<0x128>(v);
    v = v + dpp<0x124>(v);
    v = v + dpp<0x4E>(v);
    return v + dpp<0xB1>(v);
}
// the four rows' values (lanes 0, 16, 32, 48) combined into one wave-uniform value
__device__ __forceinline__ float rows_max(float v) {
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}
__device__ __forceinline__ float rows_sum(float v) {
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}
// wave-wide max / sum, uniform across the wave
__device__ __forceinline__ float wave_max(float v) { return rows_max(row16_max(v)); }
__device__ __forceinline__ float wave_sum(float v) { return rows_sum(row16_sum(v)); }

// v of lane (lane ^ m): DPP for m = 1, 2, 4, 8 (4: row_ror:4 for lanes with bit 2 set, row_ror:12 for the others); for 16
// and 32 gfx950's v_permlane16_swap / v_permlane32_swap of v with itself, whose two results hold, lane by lane, the rows
// (16) or halves (32) of v unchanged and exchanged (checked on MI355X lane by lane).
__device__ __forceinline__ float lane_xor(float v, int m, int lane) {
    const int b = __float_as_int(v);
    switch (m) {
        case 1: return dpp<0xB1>(v);
        case 2: return dpp<0x4E>(v);
        case 4: { const float a = dpp<0x124>(v), c = dpp<0x12C>(v); return (lane & 4) ? a : c; }
        case 8: return dpp<0x128>(v);
        case 16: { const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false); return __int_as_float((lane & 16) ? r[0] : r[1]); }
        default: { const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false); return __int_as_float((lane & 32) ? r[0] : r[1]); }
    }
}

// max over the workgroup; red: >= 16 floats of LDS. Ends with a barrier (red may be reused after it).
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float m = 0.f;
    for (int i = 0; i < nw; ++i) m = fmaxf(m, red[i]);
    __syncthreads();
    return m;
}

// --------------------------------------------------------------------------------------------------- block Walsh in LDS
// A row of K FP32 values lives in LDS at logical index i -> physical slot lds_slot(i) (one padding word per 32: strided
// groups of up to 32 contiguous elements and unit-stride lanes both spread over all banks).
__device__ __forceinline__ int lds_slot(int i) { return i + (i >> 5); }
__host__ __device__ __forceinline__ int lds_words(int K) { return K + (K >> 5) + 1; }

// R radix-2 stages on 2^R register values: pairs (k, k + h) for h = 1, 2, ..., 2^(R-1); the lower slot gets a + b, the upper
// a - b, exactly the butterfly of tcq_format.fwht (reference tcq_format.py:48-52), so any distribution of the pairs over lanes
// that keeps the stage order reproduces its sums bit for bit.
template <int R>
__device__ __forceinline__ void butterflies(float* v) {
#pragma unroll
    for (int s = 0; s < R; ++s) {
        const int h = 1 << s;
#pragma unroll
        for (int k = 0; k < (1 << R); ++k)
            if (!(k & h)) {
                const float a = v[k], b = v[k + h];
                v[k] = a + b;
                v[k + h] = a - b;
            }
    }
}

// One pass of R consecutive stages (index bits b0 .. b0 + R - 1) over the segment [off, off + w) of the LDS row. Each thread
// takes groups g = tid, tid + T, ...; group g covers the 2^R indices that differ only in those bits. On the last pass each
// finished value goes to out(i, v) (i relative to the segment) instead of back to LDS.
template <int R, bool LAST, class Out>
__device__ __forceinline__ void walsh_pass(float* lds, int off, int w, int b0, Out&& out) {
    const int T = blockDim.x, G = w >> R, lowmask = (1 << b0) - 1;
    for (int g = threadIdx.x; g < G; g += T) {
        const int i0 = ((g & ~lowmask) << R) | (g & lowmask);
        float v[1 << R];
#pragma unroll
        for (int k = 0; k < (1 << R); ++k) v[k] = lds[lds_slot(off + i0 + (k << b0))];
        butterflies<R>(v);
#pragma unroll
        for (int k = 0; k < (1 << R); ++k) {
            if (LAST) out(i0 + (k << b0), v[k]);
            else lds[lds_slot(off + i0 + (k << b0))] = v[k];
        }
    }
}

template <bool LAST, class Out>
__device__ __forceinline__ void walsh_pass_r(int r, float* lds, int off, int w, int b0, Out&& out) {
    switch (r) {
        case 1: walsh_pass<1, LAST>(lds, off, w, b0, out); break;
        case 2: walsh_pass<2, LAST>(lds, off, w, b0, out); break;
        case 3: walsh_pass<3, LAST>(lds, off, w, b0, out); break;
        case 4: walsh_pass<4, LAST>(lds, off, w, b0, out); break;
        default: walsh_pass<5, LAST>(lds, off, w, b0, out); break;
    }
}

// Unnormalised Walsh transform of one power-of-two segment (the LDS row must be complete and synchronised on entry). The
// log2(w) stages are split into passes of at most 5 bits, balanced (14 = 5 + 5 + 4, 11 = 4 + 4 + 3); a barrier separates
// passes. out(i, v) receives every finished value once. Ends without a barrier.
template <class Out>
__device__ __forceinline__ void walsh_segment(float* lds, int off, int w, Out&& out) {
    const int L = 31 - __clz(w);
    if (L == 0) {
        if (threadIdx.x == 0) out(0, lds[lds_slot(off)]);
        return;
    }
    const int passes = (L + 4) / 5;
    int b0 = 0;
    for (int p = 0; p < passes; ++p) {
        const int r = (L - b0) / (passes - p);
        if (p == passes - 1) {
            walsh_pass_r<true>(L - b0, lds, off, w, b0, out);
        } else {
            walsh_pass_r<false>(r, lds, off, w, b0, out);
            __syncthreads();
        }
        b0 += r;
    }
}

// Block Walsh over the binary decomposition of K (descending powers of two, reference tcq_format.py:26-30, 44-55): every value
// is multiplied by the FP32 constant float(1 / sqrt(w)) of its block (computed in FP64 then rounded, as
// np.float32(1.0 / math.sqrt(w)) in tcq_format.py:40). out(i, v) gets the normalised value at row index i. Blocks touch
// disjoint LDS so they need no barrier between them; the caller synchronises after the call.
template <class Out>
__device__ __forceinline__ void block_walsh(float* lds, int K, Out&& out) {
    int off = 0, rem = K;
    while (rem) {
        const int w = 1 << (31 - __clz(rem));
        const float c = (float)(1.0 / __builtin_sqrt((double)w));
        const int o = off;
        walsh_segment(lds, o, w, [&](int i, float v) { out(o + i, v * c); });
        off += w;
        rem -= w;
    }
}

// Register-resident Walsh transform of a power-of-two row held by the whole workgroup: thread t owns elements
// [16 t, 16 t + 16) (K = 16 * blockDim.x, 16 <= K <= 16384). Stages h = 1, 2, 4, 8 run inside the thread, h = 16 .. 512
// between the lanes of a wave (partner lane t ^ (h / 16)), larger h between waves through xs (LDS, >= K floats, k-major
// so every exchange is conflict-free). Every stage is the (a + b, a - b) butterfly of tcq_format.fwht in stage order, the
// lower index keeping a + b, so the result equals walsh_segment's bit for bit. Unnormalised; ends with a barrier when
// K > 1024 (xs may then be reused), otherwise touches no LDS at all.
__device__ __forceinline__ void reg_walsh16(float (&v)[16], int K, float* xs) {
    butterflies<4>(v);
    const int t = threadIdx.x, nt = K >> 4, lane = t & 63;
    // the six lane stages unrolled with a guard rather than a loop exit (an exit left the loop rolled in some kernels, with
    // lane_xor's choice of cross-lane move made at run time for every value)
#pragma unroll
    for (int s = 0; s < 6; ++s) {
        const int m = 1 << s;
        if (m < nt) {
            const bool upper = lane & m;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const float p = lane_xor(v[k], m, lane);
                v[k] = upper ? p - v[k] : v[k] + p;
            }
        }
    }
    for (int m = 64; m < nt; m <<= 1) {
#pragma unroll
        for (int k = 0; k < 16; ++k) xs[k * nt + t] = v[k];
        __syncthreads();
        const bool upper = t & m;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const float p = xs[k * nt + (t ^ m)];
            v[k] = upper ? p - v[k] : v[k] + p;
        }
        __syncthreads();
    }
}

// reg_walsh16 for a row of K = 16 nt values held by threads t < nt of a possibly wider workgroup: the same stages in the
// same order (lanes through shuffles, waves through xs); threads from nt on hold no values but meet every barrier.
__device__ __forceinline__ void reg_walsh16_part(float (&v)[16], int K, float* xs) {
    butterflies<4>(v);
    const int t = threadIdx.x, nt = K >> 4, lane = t & 63;
    const bool on = t < nt;
    // waves past the row skip the lane stages (their shuffles would only load the LDS crossbar)
    const bool wave_on = __builtin_amdgcn_readfirstlane(t & ~63) < nt;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        if (!wave_on || m >= nt) break;
        const bool upper = lane & m;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const float p = lane_xor(v[k], m, lane);
            v[k] = upper ? p - v[k] : v[k] + p;
        }
    }
    for (int m = 64; m < nt; m <<= 1) {
        if (on) {
#pragma unroll
            for (int k = 0; k < 16; ++k) xs[k * nt + t] = v[k];
        }
        __syncthreads();
        if (on) {
            const bool upper = t & m;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const float p = xs[k * nt + (t ^ m)];
                v[k] = upper ? p - v[k] : v[k] + p;
            }
        }
        __syncthreads();
    }
}

// Register + transpose Walsh engine: a power-of-two row of 2^L values held 2^LE per thread by 2^(L - LE) threads
// (2 LE <= L <= 3 LE). Three layouts give the row index of register k in thread t:
//   A (natural):  (t << LE) | k                                              -- register bits = index bits [0, LE)
//   B (middle):   t bits [0, LE) -> [0, LE), t bits [LE, ..) -> [L - LE, ..),
//                 k bits [0, MB) -> [LE, L - LE), k bits [MB, LE) -> [L - LE + MB, L)   (MB = L - 2 LE)
//   C (top):      t | (k << (L - LE))                                        -- register bits = index bits [L - LE, L)
// A pass runs the butterflies of its layout's register bits inside the thread; between passes the row goes once through
// LDS (lds_slot padding: every access of a half-wave hits 32 distinct banks). Since the passes cover index bits in
// ascending order, every stage is walsh_segment's butterfly in the same stage order and the sums are equal bit for bit.
// The index parts of t and k use disjoint bits, so lds_slot(t part | k part) = lds_slot(t part) + lds_slot(k part) and
// the k parts are compile-time offsets.
//
// Rows of 3 LE < L <= 4 LE take four passes instead (Tw::P4), each of LE index bits, with R = L - 3 LE for the last:
//   A (natural):  (t << LE) | k
//   B:            t bits [0, LE) -> [0, LE), the rest -> [2 LE, L); k -> [LE, 2 LE)
//   C:            t bits [0, 2 LE) -> [0, 2 LE), the rest -> [3 LE, L); k -> [2 LE, 3 LE)
//   D (last):     t -> [LE - R, 3 LE); k bits [0, R) -> [3 LE, L), k bits [R, LE) -> [0, LE - R) (bits whose stages are
//                 done: the pass runs butterflies over k bits [0, R) only)
template <int L, int LE>
struct Tw {
    static constexpr int E = 1 << LE, T = 1 << (L - LE), H = L - LE, MB = L - 2 * LE;
    static constexpr bool P4 = L > 3 * LE;
    static constexpr int R = L - 3 * LE, LAST = P4 ? 3 : 2;              // last pass: its bits, its layout
    static_assert(MB >= 0 && L <= 4 * LE, "register + transpose Walsh needs 2 LE <= L <= 4 LE");
    template <int X>
    __device__ static int tpart(int t) {
        if constexpr (P4)
            return X == 0 ? t << LE : X == 1 ? (t & (E - 1)) | ((t >> LE) << (2 * LE))
                 : X == 2 ? (t & (E * E - 1)) | ((t >> (2 * LE)) << (3 * LE)) : t << (LE - R);
        else
            return X == 0 ? t << LE : X == 1 ? (t & (E - 1)) | ((t >> LE) << H) : t;
    }
    template <int X>
    __host__ __device__ static constexpr int kpart(int k) {
        if constexpr (P4)
            return X == 0 ? k : X == 1 ? k << LE : X == 2 ? k << (2 * LE) : ((k & ((1 << R) - 1)) << (3 * LE)) | (k >> R);
        else
            return X == 0 ? k : X == 1 ? ((k & ((1 << MB) - 1)) << LE) | ((k >> MB) << (H + MB)) : k << H;
    }
};

// Stores the thread's values of layout X to their row slots in xs / loads them from there. Threads from 2^(L - LE) on (a
// workgroup wider than the row) hold no values: they skip every access but still meet every barrier of the engine.
template <int L, int LE, int X>
__device__ __forceinline__ void tw_put(const float (&v)[1 << LE], float* xs) {
    using W = Tw<L, LE>;
    if ((int)threadIdx.x >= W::T) return;
    const int b = lds_slot(W::template tpart<X>(threadIdx.x));
#pragma unroll
    for (int k = 0; k < W::E; ++k) xs[b + lds_slot(W::template kpart<X>(k))] = v[k];
}
template <int L, int LE, int X>
__device__ __forceinline__ void tw_get(float (&v)[1 << LE], const float* xs) {
    using W = Tw<L, LE>;
    if ((int)threadIdx.x >= W::T) return;
    const int b = lds_slot(W::template tpart<X>(threadIdx.x));
#pragma unroll
    for (int k = 0; k < W::E; ++k) v[k] = xs[b + lds_slot(W::template kpart<X>(k))];
}

// Unnormalised Walsh of the row held in layout A (v: the thread's 2^LE values); leaves it in layout C. xs: lds_words(2^L)
// floats. On entry no other thread may still read the thread's layout-A slots (a barrier, or only the thread itself read
// them last); on exit the thread may rewrite its own layout-C slots at once, any other slot only after a barrier.
template <int L, int LE>
__device__ __forceinline__ void tw_walsh(float (&v)[1 << LE], float* xs) {
    using W = Tw<L, LE>;
    butterflies<LE>(v);
    tw_put<L, LE, 0>(v, xs);
    __syncthreads();
    if constexpr (W::P4) {                                                 // four passes: B, C, then D
        tw_get<L, LE, 1>(v, xs);
        butterflies<LE>(v);
        tw_put<L, LE, 1>(v, xs);
        __syncthreads();
        tw_get<L, LE, 2>(v, xs);
        butterflies<LE>(v);
        tw_put<L, LE, 2>(v, xs);
        __syncthreads();
        tw_get<L, LE, 3>(v, xs);
#pragma unroll
        for (int g = 0; g < (W::E >> W::R); ++g) butterflies<W::R>(v + (g << W::R));
        return;
    }
    if constexpr (W::MB > 0) {
        tw_get<L, LE, 1>(v, xs);
#pragma unroll
        for (int g = 0; g < (W::E >> W::MB); ++g) butterflies<W::MB>(v + (g << W::MB));
        tw_put<L, LE, 1>(v, xs);
        __syncthreads();
    }
    tw_get<L, LE, 2>(v, xs);
    butterflies<LE>(v);
}

// Two independent rows at once (a in xa, b in xb: two lds_words(2^L) regions), as tw_walsh on each: one barrier per pass
// for both, and twice the independent work between barriers.
template <int L, int LE>
__device__ __forceinline__ void tw_walsh2(float (&a)[1 << LE], float (&b)[1 << LE], float* xa, float* xb) {
    using W = Tw<L, LE>;
    static_assert(!W::P4, "two rows at once: three-pass rows");
    butterflies<LE>(a);
    butterflies<LE>(b);
    tw_put<L, LE, 0>(a, xa);
    tw_put<L, LE, 0>(b, xb);
    __syncthreads();
    if constexpr (W::MB > 0) {
        tw_get<L, LE, 1>(a, xa);
        tw_get<L, LE, 1>(b, xb);
#pragma unroll
        for (int g = 0; g < (W::E >> W::MB); ++g) {
            butterflies<W::MB>(a + (g << W::MB));
            butterflies<W::MB>(b + (g << W::MB));
        }
        tw_put<L, LE, 1>(a, xa);
        tw_put<L, LE, 1>(b, xb);
        __syncthreads();
    }
    tw_get<L, LE, 2>(a, xa);
    tw_get<L, LE, 2>(b, xb);
    butterflies<LE>(a);
    butterflies<LE>(b);
}

// Walsh of a row of 2^(LE + 6) * NWP values held 2^LE per thread by waves 0 .. NWP - 1 (NWP = 4 or 8; thread t = 64 w + l:
// values 2^LE t .. in natural layout, which they keep): index bits [0, LE) inside the thread, [LE, LE + 6) across the
// lanes (lane_xor), the last log2(NWP) across the waves through xs (2^LE * 64 * NWP floats of LDS, value k of thread (w, l)
// at [(NWP k + w) * 64 + l]) after one sync() (a barrier these waves meet; a caller's other waves may meet it too). Each
// wave evaluates the butterflies its own values need (wave-uniform choices). Every stage is the (a + b, a - b) butterfly in
// ascending stage order, as in tw_walsh, so the sums are equal bit for bit. xs may be written again once every wave has
// passed a later sync().
template <int LE>
__device__ __forceinline__ void wave_walsh_lanes(float (&v)[1 << LE]) {
    constexpr int E = 1 << LE;
    butterflies<LE>(v);
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int s = 0; s < 6; ++s) {
        const int m = 1 << s;
        const bool upper = lane & m;
#pragma unroll
        for (int k = 0; k < E; ++k) {
            const float p = lane_xor(v[k], m, lane);
            v[k] = upper ? p - v[k] : v[k] + p;
        }
    }
}
template <int LE, int NWP>
__device__ __forceinline__ void wave_walsh_put(const float (&v)[1 << LE], float* xs) {
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int k = 0; k < (1 << LE); ++k) xs[(NWP * k + w) * 64 + lane] = v[k];
}
template <int LE, int NWP>
__device__ __forceinline__ void wave_walsh_get(float (&v)[1 << LE], const float* xs) {
    static_assert(NWP == 4 || NWP == 8, "four or eight waves");
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int k = 0; k < (1 << LE); ++k) {
        const float* xk = xs + NWP * k * 64 + lane;
        // y1(j): stage 1 value at wave position j (lower keeps a + b, upper gets a - b of lower a, upper b)
        auto y1 = [&](int j) {
            const float a = xk[64 * (j & ~1)], b = xk[64 * (j | 1)];
            return (j & 1) ? a - b : a + b;
        };
        auto y2 = [&](int j) {
            const float a = y1(j & ~2), b = y1(j | 2);
            return (j & 2) ? a - b : a + b;
        };
        if constexpr (NWP == 4) {
            v[k] = y2(w);
        } else {
            const float a = y2(w & ~4), b = y2(w | 4);
            v[k] = (w & 4) ? a - b : a + b;
        }
    }
}
template <int LE, int NWP, class SY>
__device__ __forceinline__ void wave_walsh(float (&v)[1 << LE], float* xs, SY&& sync) {
    wave_walsh_lanes<LE>(v);
    wave_walsh_put<LE, NWP>(v, xs);
    sync();
    wave_walsh_get<LE, NWP>(v, xs);
}
// two rows at once (a through xa, b through xb), one sync() for both
template <int LE, int NWP, class SY>
__device__ __forceinline__ void wave_walsh2(float (&a)[1 << LE], float (&b)[1 << LE], float* xa, float* xb, SY&& sync) {
    wave_walsh_lanes<LE>(a);
    wave_walsh_lanes<LE>(b);
    wave_walsh_put<LE, NWP>(a, xa);
    wave_walsh_put<LE, NWP>(b, xb);
    sync();
    wave_walsh_get<LE, NWP>(a, xa);
    wave_walsh_get<LE, NWP>(b, xb);
}

// Last layout (C, or D for four passes) -> layout A through xs (own slots first, one barrier).
template <int L, int LE>
__device__ __forceinline__ void tw_to_natural(float (&v)[1 << LE], float* xs) {
    tw_put<L, LE, Tw<L, LE>::LAST>(v, xs);
    __syncthreads();
    tw_get<L, LE, 0>(v, xs);
}

template <int L, int LE>
__device__ __forceinline__ void tw_to_natural2(float (&a)[1 << LE], float (&b)[1 << LE], float* xa, float* xb) {
    tw_put<L, LE, 2>(a, xa);
    tw_put<L, LE, 2>(b, xb);
    __syncthreads();
    tw_get<L, LE, 0>(a, xa);
    tw_get<L, LE, 0>(b, xb);
}

// ---------------------------------------------------------------------------------------------------- activation quantizer
// Per-token symmetric INT8 of tcq_format.quantize_tokens (reference tcq_format.py:119-122): the correctly rounded quotient
// v / s, rounded half-even, clamped. The quotient: for a scale in [2^-90, 2^90] (every row whose largest magnitude is a
// normal value far from overflow), q = v * (1 / s) with two Markstein corrections q += (v - q s) / s, the residuals exact
// through fused multiply-adds: with a correctly rounded reciprocal, the first correction brings q within one ulp and the
// second gives the correctly rounded quotient (Markstein's theorem) wherever nothing underflows; near the bottom of the
// scale range the residual of a quotient below 2^-12 can underflow, and such a quotient rounds to 0 either way. Checked
// against IEEE division on the host over every FP32 v of a row at six scales and 1.6e8 near-tie pairs (no rounded integer
// differs; tests/native/quotient_check.c). Other scales (tiny or huge rows, infinities) divide.
struct QScale {
    float s, rcp;
    bool fast;
};
__device__ __forceinline__ QScale qscale(float s) {
    const bool fast = s >= 0x1p-90f && s <= 0x1p90f;
    return QScale{s, fast ? 1.f / s : 0.f, fast};
}
__device__ __forceinline__ int q8(float v, const QScale& S) {
    float d;
    if (S.fast) {
        d = v * S.rcp;
        float e = __builtin_fmaf(-d, S.s, v);
        d = __builtin_fmaf(e, S.rcp, d);
        e = __builtin_fmaf(-d, S.s, v);
        d = __builtin_fmaf(e, S.rcp, d);
    } else {
        d = v / S.s;
    }
    float r = __builtin_rintf(d);
    r = fminf(fmaxf(r, -127.f), 127.f);
    return (int)r;
}
__device__ __forceinline__ float token_scale(float amax) { return amax > 0.f ? amax / 127.f : 1.f; }

// Byte offset of token t, column k in the token-block layout of a K-column activation matrix (K % 16 == 0).
__device__ __forceinline__ size_t tb_offset(int t, int k, int K) {
    return ((size_t)((t >> 4) * (K >> 4) + (k >> 4)) * 16 + (t & 15)) * 16 + (k & 15);
}

// Quantize an LDS row (logical indices 0..K-1, K % 4 == 0) with scale s: q (K bytes, row-major) and / or the q4 layout
// (K/4, ldq) int32 words (4 consecutive inputs per word, token = column), as reference kernels.py:170-184.
__device__ __forceinline__ void quantize_row(const float* lds, float sc, i8* q, int* q4, int tok, int K, int ldq) {
    const QScale s = qscale(sc);
    for (int j = threadIdx.x; j < (K >> 2); j += blockDim.x) {
        const u32 word = (u32)(q8(lds[lds_slot(4 * j)], s) & 0xff) | ((u32)(q8(lds[lds_slot(4 * j + 1)], s) & 0xff) << 8) |
                         ((u32)(q8(lds[lds_slot(4 * j + 2)], s) & 0xff) << 16) | ((u32)(q8(lds[lds_slot(4 * j + 3)], s) & 0xff) << 24);
        if (q) ((u32*)q)[j] = word;
        if (q4) {
            if (ldq == TCQ_LDQ_TOKEN_BLOCKS) *(u32*)((i8*)q4 + tb_offset(tok, 4 * j, K)) = word;
            else q4[(size_t)j * ldq + tok] = (int)word;
        }
    }
}


// ------------------------------------------------------------------------------------------------------------- trellis code
// One 16 x 16 tile = 32 uint16 words, 512 bits, most significant bit first; state t = bits [4t, 4t + 16) (tail-biting).
// Tile row r, weight pair p (columns 2p, 2p + 1) has state t = 8 r + p (reference tcq_format.py:58-63).
// Code: x = (s + 1) s; table row (x >> 6) & 511; first coordinate negated when bit 15 of x is set (tcq_format.py:66-71).
// Only bits 6..15 of x are used and they depend only on s mod 2^16, so x may be computed modulo 2^16 (two states per
// v_pk_mad_u16) from any value congruent to s.
//
// Sign-folded table: entry e in 0..1023 = (e >> 9 ? -t[e & 511][0] : t[e & 511][0], t[e & 511][1]), index e = (x >> 6) & 1023.
__device__ __forceinline__ u32 code_index(u32 x) { return (x >> 6) & 1023u; }

// x = s * s + s = (s + 1) s modulo 2^16 for both 16-bit states held in w: one v_pk_mad_u16 (the compiler splits the
// vector expression into an add and a multiply)
__device__ __forceinline__ u32 pk_code(u32 w) {
    u32 x;
    asm("v_pk_mad_u16 %0, %1, %1, %1" : "=v"(x) : "v"(w));
    return x;
}

// ------------------------------------------------------------------------------------------------------- buffer loads
// Raw buffer resource over [p, p + bytes): loads address it with a 32-bit per-lane offset plus a wave-uniform offset, and a
// lane whose offset lies at or beyond `bytes` reads zeros. Word 3 = 0x00020000: 32-bit data format, no swizzle (gfx9 family).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* p, u32 bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
constexpr u32 RSRC_OOB = 0x80000000u;   // a lane offset that always reads zeros (buffers stay below 2 GiB)

// Global-address-space view of a generic pointer: loads and stores through it are global_* instructions, which count only
// on vmcnt (flat ones also count on lgkmcnt and make the compiler wait for every LDS read as well).
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gptr(T* p) {
    return (__attribute__((address_space(1))) T*)p;
}
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gptr(const T* p) {
    return (const __attribute__((address_space(1))) T*)p;
}

// Raw 16-element chunks of the side vectors, loaded at kernel entry together with the accumulator row (they do not depend
// on it) and converted where they are used, so no global round trip waits behind a Walsh pass. ESZ: element bytes (1 INT8,
// 2 BF16, 4 FP32); the raw words hold the elements little-endian, as in memory. Unaligned rows load element by element.
template <int ESZ> struct Raw16 {
    uint4_t r[ESZ];
};
template <int ESZ>
__device__ __forceinline__ Raw16<ESZ> raw16(const void* p, bool vec) {
    Raw16<ESZ> o;
    if (vec) {
#pragma unroll
        for (int q = 0; q < ESZ; ++q) o.r[q] = gptr((const uint4_t*)p)[q];
    } else {
#pragma unroll
        for (int q = 0; q < ESZ; ++q) o.r[q] = uint4_t{0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const u32 e = ESZ == 1 ? (u32)(uint8_t)gptr((const i8*)p)[k] : ESZ == 2 ? (u32)gptr((const u16*)p)[k] : gptr((const u32*)p)[k];
            const int bit = 8 * ESZ * k;                                 // bit offset of element k in the 16 * ESZ bytes
            o.r[bit >> 7][(bit >> 5) & 3] |= e << (bit & 31);
        }
    }
    return o;
}
__device__ __forceinline__ void cv16(const Raw16<1>& a, float (&v)[16]) {
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = (float)(i8)(a.r[0][k >> 2] >> (8 * (k & 3)));
}
__device__ __forceinline__ void cv16(const Raw16<2>& a, float (&v)[16]) {
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = bf16_to_f32((u16)(a.r[k >> 3][(k >> 1) & 3] >> (16 * (k & 1))));
}
__device__ __forceinline__ void cv16(const Raw16<4>& a, float (&v)[16]) {
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = __uint_as_float(a.r[k >> 2][k & 3]);
}

// Rotate + quantize of a register row (values already signed): walsh, * c, per-token absmax, INT8 words (as k_pre).
// Threads from N / 16 on (a workgroup wider than the row) hold no values: they meet the barriers and store nothing.
__device__ __forceinline__ void reg_rotate_quantize(float (&v)[16], int N, float* xs, float* red, i8* q, int* q4, int ldq,
                                                    float* scale, int tok) {
    const int t = threadIdx.x;
    const float c = (float)(1.0 / __builtin_sqrt((double)N));
    reg_walsh16_part(v, N, xs);
    float mx = 0.f;
    const bool on = t < (N >> 4);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        v[k] = v[k] * c;
        if (on) mx = fmaxf(mx, fabsf(v[k]));
    }
    const float sc = token_scale(block_max(mx, red));
    if (t == 0) scale[tok] = sc;
    if (!on) return;
    const QScale S = qscale(sc);
    u32 words[4];
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4)
        words[k4] = (u32)(q8(v[4 * k4], S) & 0xff) | ((u32)(q8(v[4 * k4 + 1], S) & 0xff) << 8) |
                    ((u32)(q8(v[4 * k4 + 2], S) & 0xff) << 16) | ((u32)(q8(v[4 * k4 + 3], S) & 0xff) << 24);
    if (q) *gptr((uint4_t*)(q + (size_t)tok * N + 16 * t)) = uint4_t{words[0], words[1], words[2], words[3]};
    if (q4 && ldq == TCQ_LDQ_TOKEN_BLOCKS) {
        *gptr((uint4_t*)((i8*)q4 + tb_offset(tok, 16 * t, N))) = uint4_t{words[0], words[1], words[2], words[3]};
    } else if (q4) {
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) q4[(size_t)(4 * t + k4) * ldq + tok] = (int)words[k4];
    }
}

// 16-element view of part h of a register array (for the 16-wide loaders and converters).
template <int E>
__device__ __forceinline__ float (&part16(float (&v)[E], int h))[16] { return *reinterpret_cast<float(*)[16]>(&v[16 * h]); }

// reg_rotate_quantize on the register + transpose engine: v holds the natural-layout values 2^LE t .. 2^LE t + 2^LE - 1 of
// the row (N = 2^L); the same operations in the same order (Walsh, * c, row max, per-token INT8, q and / or q4 words).
// Threads from 2^(L - LE) on (a workgroup wider than the row) hold no values: they meet the barriers and store nothing.
// Any of q, q4, scale may be NULL; qs / scs (LDS, optional): the row's INT8 words (word j = inputs 4j .. 4j + 3) and its
// scale are also left there.
template <int L, int LE>
__device__ __forceinline__ void tw_rotate_quantize(float (&v)[1 << LE], float* xs, float* red, i8* q, int* q4, int ldq,
                                                   float* scale, int tok, u32* qs = nullptr, float* scs = nullptr) {
    constexpr int N = 1 << L, E = 1 << LE;
    const int t = threadIdx.x;
    const bool on = t < (N >> LE);
    const float c = (float)(1.0 / __builtin_sqrt((double)N));
    tw_walsh<L, LE>(v, xs);
    float mx = 0.f;
#pragma unroll
    for (int k = 0; k < E; ++k) {
        v[k] = v[k] * c;
        if (on) mx = fmaxf(mx, fabsf(v[k]));
    }
    const float sc = token_scale(block_max(mx, red));
    if (t == 0 && scale) scale[tok] = sc;
    if (t == 0 && scs) *scs = sc;
    tw_to_natural<L, LE>(v, xs);
    if (!on) return;
    const QScale S = qscale(sc);
    u32 words[E / 4];
#pragma unroll
    for (int k4 = 0; k4 < E / 4; ++k4)
        words[k4] = (u32)(q8(v[4 * k4], S) & 0xff) | ((u32)(q8(v[4 * k4 + 1], S) & 0xff) << 8) |
                    ((u32)(q8(v[4 * k4 + 2], S) & 0xff) << 16) | ((u32)(q8(v[4 * k4 + 3], S) & 0xff) << 24);
    if constexpr (E == 8) {                                             // 8 bytes per thread: half a 16-byte group
        const u64 d = (u64)words[0] | ((u64)words[1] << 32);
        if (qs) *(u64*)(qs + 2 * t) = d;
        if (q) *gptr((u64*)(q + (size_t)tok * N + 8 * t)) = d;
        if (q4 && ldq == TCQ_LDQ_TOKEN_BLOCKS) *gptr((u64*)((i8*)q4 + tb_offset(tok, 8 * t, N))) = d;
    } else {
        if (qs) {
#pragma unroll
            for (int h = 0; h < E / 16; ++h)
                *(uint4_t*)(qs + (E / 4) * t + 4 * h) = uint4_t{words[4 * h], words[4 * h + 1], words[4 * h + 2], words[4 * h + 3]};
        }
        if (q) {
#pragma unroll
            for (int h = 0; h < E / 16; ++h)
                *gptr((uint4_t*)(q + (size_t)tok * N + E * t + 16 * h)) =
                    uint4_t{words[4 * h], words[4 * h + 1], words[4 * h + 2], words[4 * h + 3]};
        }
        if (q4 && ldq == TCQ_LDQ_TOKEN_BLOCKS) {
#pragma unroll
            for (int h = 0; h < E / 16; ++h)
                *gptr((uint4_t*)((i8*)q4 + tb_offset(tok, E * t + 16 * h, N))) =
                    uint4_t{words[4 * h], words[4 * h + 1], words[4 * h + 2], words[4 * h + 3]};
        }
    }
    if (q4 && ldq != TCQ_LDQ_TOKEN_BLOCKS) {
#pragma unroll
        for (int k4 = 0; k4 < E / 4; ++k4) q4[(size_t)((E / 4) * t + k4) * ldq + tok] = (int)words[k4];
    }
}

// Coalesced loading / storing of a wave's span of a row (elements of ESZ = 2 or 4 bytes): the wave's threads hold the
// 64 * 2^LE values [64 w 2^LE, 64 (w + 1) 2^LE) in layout A, and moving them thread by thread (2^LE * ESZ bytes per lane)
// makes every memory instruction touch up to 64 cache lines. Instead lane l moves the 16-byte pieces 64 j + l of the span,
// so each instruction covers one contiguous KiB, and the values pass through their row slots in xs. A piece holds
// 16 / ESZ consecutive values, which never straddle a padding word; the lanes of a half-wave hit 32 distinct banks.
template <int LE, int ESZ>
struct Span {
    uint4_t p[(1 << LE) * ESZ / 16];
};
template <int LE, int ESZ>
__device__ __forceinline__ Span<LE, ESZ> tw_span_load(const void* row) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint4_t* s = (const uint4_t*)((const char*)row + ((size_t)w << (LE + 6)) * ESZ);
    Span<LE, ESZ> r;
#pragma unroll
    for (int j = 0; j < (1 << LE) * ESZ / 16; ++j) r.p[j] = *gptr(s + 64 * j + lane);
    return r;
}
// xs slot of value m of piece j; f(j, m, bits) converts the raw bits of a value (ESZ = 2: the low 16 bits)
template <int LE, int ESZ>
__device__ __forceinline__ float* tw_piece_slot(float* xs, int j) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    return xs + lds_slot((w << (LE + 6)) + (16 / ESZ) * (64 * j + lane));
}
template <int LE, int ESZ, class F>
__device__ __forceinline__ void tw_span_put(const Span<LE, ESZ>& r, float* xs, F&& f) {
#pragma unroll
    for (int j = 0; j < (1 << LE) * ESZ / 16; ++j) {
        float* d = tw_piece_slot<LE, ESZ>(xs, j);
#pragma unroll
        for (int m = 0; m < 16 / ESZ; ++m)
            d[m] = f(j, m, ESZ == 4 ? r.p[j][m] : (r.p[j][m >> 1] >> (16 * (m & 1))) & 0xffffu);
    }
}
// the span from its row slots to memory as YDT (F32, BF16 or F16)
template <int LE, int YDT>
__device__ __forceinline__ void tw_span_store(void* row, float* xs) {
    constexpr int ESZ = YDT == TCQ_F32 ? 4 : 2;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    uint4_t* o = (uint4_t*)((char*)row + ((size_t)w << (LE + 6)) * ESZ);
    constexpr int NJ = (1 << LE) * ESZ / 16;
    if constexpr (YDT == TCQ_BF16) {                                     // every piece converted in one batch
        float d[8 * NJ];
        u32 w[4 * NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) d[8 * j + e] = tw_piece_slot<LE, ESZ>(xs, j)[e];
        bf16_pack<4 * NJ>(d, w);
#pragma unroll
        for (int j = 0; j < NJ; ++j) *gptr(o + 64 * j + lane) = uint4_t{w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]};
        return;
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const float* d = tw_piece_slot<LE, ESZ>(xs, j);
        uint4_t v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            v[e] = YDT == TCQ_F32 ? __float_as_uint(d[e]) : (u32)f32_to_f16(d[2 * e]) | ((u32)f32_to_f16(d[2 * e + 1]) << 16);
        *gptr(o + 64 * j + lane) = v;
    }
}
