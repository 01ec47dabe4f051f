// Attention shapes and the chunk merge shared by the attention kernels (tcq_attend.hip) and the products that run the
// merge as their prologue (tcq_gemm_small.hip).
#pragma once
#include "tcq_device.h"

constexpr int AD = 256;          // head dim
constexpr int AH = 8;            // most query heads
constexpr int KC = 64;           // keys per chunk
constexpr int PS = AD + 4;       // floats per (token, chunk, head) partial: o[AD], m, l and 2 pad words (16-byte rows)
constexpr int MAXC = 256;        // most chunks a token may have in the combine (16384 keys)
constexpr int CW = 16;           // chunks whose values a lane loads at entry in combine_w_row

// Chunks of token t that hold a key it sees: the combine merges only these. A chunk past them has m = -inf, l = 0 and o = 0
// for t (weight 0), and adding 0 * 0 to a sum that starts at +0 changes no bit, so skipping them gives the same result;
// k_attn_part does not compute the chunks no token of its group sees.
__device__ __forceinline__ int visible_chunks(int NC, int T, int causal, int t) {
    return causal >= 0 ? min(NC, (min(T, causal + t + 1) + KC - 1) / KC) : NC;
}

// The merge of token t's chunk partials (part: (M, NC, H, PS) FP32 from k_attn_part), one wave per head: lane l of wave
// h < H owns dims 4 l .. 4 l + 3 of head h and loads them for the first CW chunks together with the chunk statistics at
// entry. Every 16-lane group repeats the statistics merge (lane g: chunks g, g + 16, ...; a butterfly over the 16 lanes),
// and the chunks add in chunk order, so the result depends only on the chunking. o (optional): the BF16 row. With su, the
// BF16 row times su goes to xs (natural slots) for the rotate + quantize that follows, and the function ends with a
// barrier; without su it returns false (uniform) and there is no barrier. Waves from H on take no part in the merge.
// mid() runs once the entry loads have been consumed.
// vr (H = 8): instead of xs, the thread's four values (dims 4 l .. of head h: row values 4 tid ..) go to vr, with no barrier.
template <class F>
__device__ __forceinline__ bool combine_w_row(const float* part, int NC, int T, int causal, int H, int t, u16* o, const i8* su,
                                              float* xs, float (*wts)[MAXC], F&& mid, float* vr = nullptr) {
    const int tid = threadIdx.x, h = tid >> 6, lane = tid & 63, g = lane & 15, d0 = 4 * lane, K = H * AD;
    const bool on = h < H;                                               // whole waves
    const size_t cs = (size_t)H * PS;
    const float* hb = part + (size_t)t * NC * cs + (size_t)(on ? h : 0) * PS;   // head h of chunk 0
    const int NV = visible_chunks(NC, T, causal, t);
    constexpr int SC = MAXC / 16;
    typedef float f2_t __attribute__((ext_vector_type(2)));
    f2_t ml[SC];
    float4_t v[CW];
#pragma unroll
    for (int r = 0; r < SC; ++r) {
        const int c = g + 16 * r;
        ml[r] = (on && c < NV) ? gptr((const f2_t*)(hb + c * cs + AD))[0] : f2_t{-__builtin_inff(), 0.f};
    }
#pragma unroll
    for (int i = 0; i < CW; ++i) v[i] = (on && i < NV) ? gptr((const float4_t*)(hb + i * cs + d0))[0] : float4_t{0.f, 0.f, 0.f, 0.f};
    float mx = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < SC; ++r) mx = fmaxf(mx, ml[r].x);
    mx = row16_max(mx);
    float L = 0.f;
#pragma unroll
    for (int r = 0; r < SC; ++r) {
        const int c = g + 16 * r;
        if (on && c < NV) {
            const float w = ml[r].x == -__builtin_inff() ? 0.f : expf(ml[r].x - mx);
            if (lane < 16) wts[h][c] = w;                                // read back by this wave only: LDS keeps its order
            L = __builtin_fmaf(w, ml[r].y, L);
        }
    }
    L = row16_sum(L);
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < CW; ++i) {
        if (on && i < NV) {
            const float w = wts[h][i];
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[k] = __builtin_fmaf(w, v[i][k], acc[k]);
        }
    }
    for (int c = CW; on && c < NV; ++c) {
        const float4_t vc = gptr((const float4_t*)(hb + c * cs + d0))[0];
        const float w = wts[h][c];
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[k] = __builtin_fmaf(w, vc[k], acc[k]);
    }
    mid();
    u16 b[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) b[k] = f32_to_bf16(acc[k] / L);
    if (on && o) *gptr((u64*)(o + (size_t)t * K + h * AD + d0)) = (u64)b[0] | ((u64)b[1] << 16) | ((u64)b[2] << 32) | ((u64)b[3] << 48);
    if (!su) return false;                                               // uniform
    if (vr) {                                                            // the caller's registers: values 4 tid .. 4 tid + 3
        const u32 sg = on ? *gptr((const u32*)(su + h * AD + d0)) : 0u;
#pragma unroll
        for (int k = 0; k < 4; ++k) vr[k] = bf16_to_f32(b[k]) * (float)(i8)(sg >> (8 * k));
        return true;
    }
    if (on) {
        const u32 sg = *gptr((const u32*)(su + h * AD + d0));
#pragma unroll
        for (int k = 0; k < 4; ++k) xs[lds_slot(h * AD + d0 + k)] = bf16_to_f32(b[k]) * (float)(i8)(sg >> (8 * k));
    }
    __syncthreads();
    return true;
}
