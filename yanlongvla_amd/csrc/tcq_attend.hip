// Attention of H query heads over one shared key / value head (multi-query, head dim 256), BF16 in and out, FP32
// arithmetic: the attention of the Gemma decoder layers whose projections run on the TCQ kernels. The keys are the cache
// rows followed by this call's own rows, so no concatenated copy is made.
//
// Split over the keys (64 per chunk): k_attn_part computes, for a group of query tokens and one key chunk, the scores of every
// head (BF16 MFMA, FP32 sums), their chunk maximum m, the exponentials e = exp(s - m), l = sum e (FP32) and the unnormalised
// outputs o = sum bf16(e) v (BF16 MFMA, FP32 sums); then
// k_attn_combine merges the chunks of a token (weights exp(m_c - max_c m_c)) and divides by the merged sum. The result
// depends on the number of keys only through this fixed chunking, never on launch shapes. The combine can feed its BF16
// output row straight into the rotate + quantize prologue of the output projection. The dot products and weighted sums
// use fused multiply-adds (this attention is the decoder layers' own definition, not a reference rounding chain).
#include "tcq_device.h"
#include "tcq_launch.h"
#include "tcq_attend.h"
#include "tcq_rows.h"

namespace {

constexpr int AT = 256;          // threads of k_attn_part

__device__ __forceinline__ const u16* key_row(const u16* cache, const u16* fresh, int P, int j) {
    return j < P ? cache + (size_t)j * AD : fresh + (size_t)(j - P) * AD;
}

}  // namespace

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
constexpr int VST = 272;          // u16 stride of the staged value rows: 136 words, so keys lg + 4i of lane groups lg = 0..3 fall
                                  // 8 banks apart and a 16-lane x 2-byte fragment read is free of conflicts

__device__ __forceinline__ float4_t mma_bf16(uint4_t a, uint4_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// grid (token groups ceil(M / TPB), chunks NC), AT = 256 threads (4 waves). part: (M, NC, H, PS) FP32: o[AD], m, l per
// head. The query rows of the group (row r = token TPB x + r / 8, head r % 8; zero rows for heads >= H and tokens >= M) form
// RB = TPB / 2 blocks of 16 MFMA rows, staged once in LDS, so one staged chunk of keys / values serves TPB tokens (the keys
// and values are the bulk of the traffic: every group reads every chunk).
// Scores on v_mfma_f32_16x16x32_bf16: A = 16 query rows, B = 16 keys per wave, 8 K steps of 32 dims; lane (g, c) of D holds
// rows 4 g .. 4 g + 3 of key c. Each row is masked with its own token's causal bound. Softmax statistics per row over the
// chunk's 64 keys. Outputs on the same MFMA: A = the exponentials e (BF16, rows x keys), B = 16 value columns x 32 keys
// gathered from the LDS stage; each wave owns 4 of the 16 column tiles, 2 K steps. Element i of lane group lg in K step ks
// is key 32 ks + lg + 4 i in both operands (any common order of the K index gives the same product).
// The q / k / v epilogue of a one-token FP32 product row, run by k_attn_part<2, true> instead of a separate launch: the
// output rotations y = bf16((walsh(z) * c) * sv), c = 1 / sqrt(n), of the q segment (8 heads x 256, 2048 wide) in every
// workgroup and of the new key / value rows (256 wide each) in the workgroup whose chunk holds key P, which also stores
// them at k_out / v_out (the cache row P). The same stages in the same order as the epilogue kernel (k_postg_tw), so the
// same bits.
struct AttnPost {
    const float* zq;
    const float* zk;
    const float* zv;
    const i8* sq;
    const i8* sk;
    const i8* sv;
    u16* k_out;
    u16* v_out;
};

// POST (M = 1, H = 8): q, kn and vn are not read; the query row and the new key / value row come from AttnPost.
template <int TPB, bool POST = false>
__global__ __launch_bounds__(AT) void k_attn_part(const u16* q, const u16* kc, const u16* vc, int P, const u16* kn, const u16* vn,
                                                  int M, int H, int causal, float* part, AttnPost ap) {
    constexpr int AR = 8 * TPB, RB = AR / 16, QST = AD + 8;       // query rows, MFMA row blocks, padded row stride (u16)
    constexpr int QW = 2048 + 64 + 1;                             // lds_words(2048): the q rotation's exchange row
    __shared__ float ps[AR][KC + 1];
    __shared__ __attribute__((aligned(16))) u16 vs[KC][VST];
    __shared__ __attribute__((aligned(16))) u16 qs[AR][QST];
    __shared__ float xq[POST ? QW : 1];
    __shared__ __attribute__((aligned(16))) u16 kns[POST ? AD : 8];
    const int t0 = TPB * blockIdx.x, c = blockIdx.y, NC = gridDim.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int T = P + M, j0 = c * KC;
    auto visible_end = [&](int t) { return min(T, causal >= 0 ? causal + t + 1 : T); };   // keys j < end are visible to t
    const int jend = visible_end(min(t0 + TPB, M) - 1);                 // the group's last token sees the most keys
    const float scl = 1.f / 16.f;                                       // 1 / sqrt(256), exact
    const bool fresh = POST && j0 <= P && P < j0 + KC;                  // POST: this workgroup makes the new key / value row
    if (j0 >= jend && !fresh) return;                                   // no key of the chunk is visible to the group; the
                                                                        // combine never reads its slots (visible_chunks)
    // POST: this thread's 8 values of the q segment and their signs, and (waves 0 and 1 of the fresh workgroup) 4 values of
    // the key (wave 0) or value (wave 1) segment per lane, issued first
    float zq[8] = {}, zr[4] = {};
    u64 gq = 0;
    u32 gr = 0;
    const bool kvw = fresh && wave < 2;                                 // wave-uniform
    if constexpr (POST) {
        const uint4_t* zp = (const uint4_t*)(ap.zq + 8 * tid);
        const uint4_t a = gptr(zp)[0], b = gptr(zp)[1];
#pragma unroll
        for (int k = 0; k < 4; ++k) { zq[k] = __uint_as_float(a[k]); zq[4 + k] = __uint_as_float(b[k]); }
        gq = gptr((const u64*)(ap.sq + 8 * tid))[0];
        if (kvw) {
            const float4_t r = gptr((const float4_t*)((wave ? ap.zv : ap.zk) + 4 * lane))[0];
#pragma unroll
            for (int k = 0; k < 4; ++k) zr[k] = r[k];
            gr = gptr((const u32*)((wave ? ap.sv : ap.sk) + 4 * lane))[0];
        }
    }
    // value stage (64 rows x 256 dims, 8 granules of 16 bytes per thread) and query rows (AR x 256), issued first (POST:
    // the new row P is staged by its maker below)
    uint4_t vg[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int gi = u * AT + tid, row = gi >> 5, col = gi & 31, j = j0 + row;
        vg[u] = j < jend && !(POST && j >= P) ? gptr((const uint4_t*)(key_row(vc, vn, P, j) + 8 * col))[0] : uint4_t{0, 0, 0, 0};
    }
    constexpr int QG = AR * 32 / AT;                                    // 16-byte query granules per thread
    uint4_t qg[QG];
#pragma unroll
    for (int u = 0; u < QG; ++u) {
        const int gi = u * AT + tid, row = gi >> 5, col = gi & 31, t = t0 + (row >> 3), h = row & 7;
        qg[u] = (!POST && h < H && t < M) ? gptr((const uint4_t*)(q + ((size_t)t * H + h) * AD + 8 * col))[0] : uint4_t{0, 0, 0, 0};
    }
    // this lane's key (B column) for the scores: its 8 fragments straight into registers (POST: the new key from LDS later)
    const int jk = j0 + 16 * wave + lr;
    const bool kv = jk < jend;
    const bool kl = kv && !(POST && jk >= P);
    const u16* kr = kl ? key_row(kc, kn, P, jk) : nullptr;
    uint4_t B[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) B[ks] = kl ? gptr((const uint4_t*)(kr + 32 * ks + 8 * lg))[0] : uint4_t{0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < QG; ++u) {
        const int gi = u * AT + tid;
        if (!POST || (gi >> 5) >= 8) *(uint4_t*)&qs[gi >> 5][8 * (gi & 31)] = qg[u];   // POST: rows 0 .. 7 made below
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int gi = u * AT + tid;
        if (!(fresh && j0 + (gi >> 5) == P)) *(uint4_t*)&vs[gi >> 5][8 * (gi & 31)] = vg[u];
    }
    if constexpr (POST) {
        if (kvw) {                                                      // the new key (wave 0) / value (wave 1) row, in the wave:
            butterflies<2>(zr);                                         // h = 1, 2 in the lane, h = 4 .. 128 across the lanes
#pragma unroll
            for (int s = 0; s < 6; ++s) {
                const int m = 1 << s;
                const bool upper = lane & m;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float pv = lane_xor(zr[k], m, lane);
                    zr[k] = upper ? pv - zr[k] : zr[k] + pv;
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) zr[k] = (zr[k] * scl) * (float)(i8)(gr >> (8 * k));   // c = 1 / sqrt(256)
            u32 w2[2];
            bf16_pack<2>(zr, w2);
            const u64 d = (u64)w2[0] | ((u64)w2[1] << 32);
            gptr((u64*)((wave ? ap.v_out : ap.k_out) + 4 * lane))[0] = d;
            if (wave == 0) *(u64*)&kns[4 * lane] = d;
            else *(u64*)&vs[P - j0][4 * lane] = P < jend ? d : 0ull;
        }
        if (fresh && j0 >= jend) return;                                // uniform: no visible key in the chunk
        // the query row on the no-transpose engine: index bits inside the thread, across the lanes, across the 4 waves
        wave_walsh<3, 4>(zq, xq, [] { __syncthreads(); });
        const float cq = (float)(1.0 / __builtin_sqrt(2048.0));
#pragma unroll
        for (int k = 0; k < 8; ++k) zq[k] = zq[k] * cq;
#pragma unroll
        for (int k = 0; k < 8; ++k) zq[k] = zq[k] * (float)(i8)(gq >> (8 * k));
        u32 w[4];
        bf16_pack<4>(zq, w);
        *(uint4_t*)&qs[tid >> 5][8 * (tid & 31)] = uint4_t{w[0], w[1], w[2], w[3]};   // head tid / 32, dims 8 (tid % 32) ..
    }
    __syncthreads();
    if (POST && kv && jk >= P) {                                        // the new key's fragments, staged above
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) B[ks] = *(const uint4_t*)&kns[32 * ks + 8 * lg];
    }
    // scores of every row block against this wave's 16 keys
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) acc = mma_bf16(*(const uint4_t*)&qs[16 * rb + lr][32 * ks + 8 * lg], B[ks], acc);
        const bool vis = jk < visible_end(t0 + 2 * rb + (lg >> 1));      // rows 16 rb + 4 lg .. + 3: token t0 + 2 rb + lg / 2
#pragma unroll
        for (int e = 0; e < 4; ++e) ps[16 * rb + 4 * lg + e][16 * wave + lr] = vis ? acc[e] * scl : -__builtin_inff();
    }
    __syncthreads();
    // chunk softmax statistics: wave w takes rows w, w + 4, ..., lane = key; the rows' reductions run side by side (each
    // row's own order unchanged), so their cross-lane exchanges overlap instead of forming one long dependent chain
    constexpr int RW = AR / 4;
    float sv[RW], m[RW], e[RW], l[RW];
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) m[rr] = sv[rr] = ps[4 * rr + wave][lane];
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) m[rr] = row16_max(m[rr]);
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) m[rr] = rows_max(m[rr]);
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) l[rr] = e[rr] = m[rr] == -__builtin_inff() ? 0.f : expf(sv[rr] - m[rr]);
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) l[rr] = row16_sum(l[rr]);
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) l[rr] = rows_sum(l[rr]);
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) {
        const int r = 4 * rr + wave, t = t0 + (r >> 3), h = r & 7;
        ps[r][lane] = e[rr];
        if (lane == 0 && h < H && t < M) {
            float* base = part + (((size_t)t * NC + c) * H + h) * PS;
            base[AD] = m[rr];
            base[AD + 1] = l[rr];
        }
    }
    __syncthreads();
    // unnormalised outputs o[r][d] = sum_k e[r][k] v[k][d]
    uint4_t A[RB][2];                                                   // e of row 16 rb + lr, BF16
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            u32 w[4];
#pragma unroll
            for (int k2 = 0; k2 < 4; ++k2) {
                const int k0 = 32 * ks + lg + 8 * k2;                   // elements 2 k2, 2 k2 + 1: keys k0, k0 + 4
                w[k2] = bf16x2(ps[16 * rb + lr][k0], ps[16 * rb + lr][k0 + 4]);
            }
            A[rb][ks] = uint4_t{w[0], w[1], w[2], w[3]};
        }
#pragma unroll
    for (int tl = 0; tl < 4; ++tl) {
        const int d = 16 * (4 * wave + tl) + lr;                         // this lane's value column
        uint4_t Bv[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            u32 w[4];
#pragma unroll
            for (int k2 = 0; k2 < 4; ++k2) {
                const int k0 = 32 * ks + lg + 8 * k2;
                w[k2] = (u32)vs[k0][d] | ((u32)vs[k0 + 4][d] << 16);
            }
            Bv[ks] = uint4_t{w[0], w[1], w[2], w[3]};
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) acc = mma_bf16(A[rb][ks], Bv[ks], acc);
            const int t = t0 + 2 * rb + (lg >> 1);
            if (t < M) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int h = 4 * (lg & 1) + e;
                    if (h < H) part[(((size_t)t * NC + c) * H + h) * PS + d] = acc[e];
                }
            }
        }
    }
}

// grid M, CT = 1024 threads: thread (d, g) = (tid % 256, tid / 256) sums dim d of every head over the chunks c = g (mod 4);
// wave h < H first merges head h's chunk statistics (lane = chunk). The four partial sums of a head add in the fixed order
// ((g0 + g1) + g2) + g3, so the result depends only on NC. With su set, the BF16 row (H x 256) is rotated and quantized
// in place as the output projection's prologue.
constexpr int CT = 1024, CG = CT / AD, CB = 4;   // threads, chunk groups, chunks per group held in registers per batch

__global__ __launch_bounds__(CT) void k_attn_combine(const float* part, int NC, int T, int causal, int H, u16* o, const i8* su, i8* q8,
                                                     int* q4, int ldq, float* scale) {
    extern __shared__ float lds[];
    __shared__ float red[CT / 64];
    __shared__ float wts[AH][MAXC];
    __shared__ float inv[AH];
    __shared__ float sums[CG][AH][AD];
    const int t = blockIdx.x, tid = threadIdx.x, d = tid & (AD - 1), g = tid / AD, lane = tid & 63, wave = tid >> 6, K = H * AD;
    const size_t cs = (size_t)H * PS;                          // stride between chunks
    const float* tb = part + (size_t)t * NC * cs;
    const int NV = visible_chunks(NC, T, causal, t);
    constexpr int SR = MAXC / 64;
    float mv[SR], lv[SR];
    if (wave < H) {
#pragma unroll
        for (int r = 0; r < SR; ++r) {
            const int c = 64 * r + lane;
            mv[r] = c < NV ? tb[c * cs + wave * PS + AD] : -__builtin_inff();
            lv[r] = c < NV ? tb[c * cs + wave * PS + AD + 1] : 0.f;
        }
    }
    float v[CB][AH];
    auto load = [&](int c0) {
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int c = c0 + g + CG * i;
#pragma unroll
            for (int h = 0; h < AH; ++h) v[i][h] = c < NV && h < H ? tb[c * cs + h * PS + d] : 0.f;
        }
    };
    load(0);
    if (wave < H) {
        float mx = -__builtin_inff();
#pragma unroll
        for (int r = 0; r < SR; ++r) mx = fmaxf(mx, mv[r]);
        mx = wave_max(mx);
        float L = 0.f;
#pragma unroll
        for (int r = 0; r < SR; ++r) {
            const int c = 64 * r + lane;
            const float w = mv[r] == -__builtin_inff() ? 0.f : expf(mv[r] - mx);
            if (c < NV) wts[wave][c] = w;
            L = __builtin_fmaf(w, lv[r], L);
        }
        L = wave_sum(L);
        if (lane == 0) inv[wave] = L;
    }
    __syncthreads();
    float acc[AH];
#pragma unroll
    for (int h = 0; h < AH; ++h) acc[h] = 0.f;
    for (int c0 = 0; c0 < NV; c0 += CG * CB) {
        if (c0) load(c0);
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int c = c0 + g + CG * i;
            if (c < NV) {
#pragma unroll
                for (int h = 0; h < AH; ++h)
                    if (h < H) acc[h] = __builtin_fmaf(wts[h][c], v[i][h], acc[h]);
            }
        }
    }
#pragma unroll
    for (int h = 0; h < AH; ++h)
        if (h < H) sums[g][h][d] = acc[h];
    __syncthreads();
#pragma unroll
    for (int hh = 0; hh < AH / CG; ++hh) {
        const int h = (AH / CG) * g + hh;
        if (h < H) {
            const float tot = ((sums[0][h][d] + sums[1][h][d]) + sums[2][h][d]) + sums[3][h][d];
            const u16 b = f32_to_bf16(tot / inv[h]);
            if (o) gptr(o)[(size_t)t * K + h * AD + d] = b;
            if (su) lds[lds_slot(h * AD + d)] = bf16_to_f32(b) * (float)gptr(su)[h * AD + d];
        }
    }
    if (!su) return;
    __syncthreads();
    float amx = 0.f;
    block_walsh(lds, K, [&](int i, float v) { lds[lds_slot(i)] = v; amx = fmaxf(amx, fabsf(v)); });
    const float sc = token_scale(block_max(amx, red));
    if (threadIdx.x == 0) scale[t] = sc;
    quantize_row(lds, sc, q8 ? q8 + (size_t)t * K : nullptr, q4, t, K, ldq);
}

// rotate + quantize of the combined row (2^L values in xs, natural layout) on the register + transpose engine, 8 values per
// thread on threads 0 .. 2^(L - 3) - 1 (one row per workgroup: more threads per row shorten it); the rest of the
// workgroup meets the barriers
template <int L>
__device__ __forceinline__ void combine_rotate_quantize(float* xs, float* red, i8* q8, int* q4, int ldq, float* scale, int t) {
    float v[8];
    tw_get<L, 3, 0>(v, xs);
    tw_rotate_quantize<L, 3>(v, xs, red, q8, q4, ldq, scale, t);
}
// grid M, H * 64 threads (one wave per head, H <= 8): lane l of wave h owns dims 4 l .. 4 l + 3 of head h and loads them for
// the first CW chunks together with the chunk statistics at entry, so a token of up to CW chunks costs one memory round trip
// (k_attn_combine_reg holds 8 chunks and goes back to memory for the rest). Every 16-lane group repeats the statistics merge
// of k_attn_combine_reg in its order (lane g: chunks g, g + 16, ...; butterfly over the 16 lanes), and the chunks add in
// chunk order, so o is the same to the bit; with su the BF16 row is rotated on the LDS Walsh engine (the same values as the
// register engine) and quantized.
__global__ __launch_bounds__(512) void k_attn_combine_w(const float* part, int NC, int T, int causal, int H, u16* o, const i8* su,
                                                        i8* q8, int* q4, int ldq, float* scale, int tw_ok) {
    extern __shared__ float xs[];                                        // lds_words(H * AD) floats: the row to rotate
    __shared__ float wts[AH][MAXC];
    __shared__ float red[16];
    __shared__ WavesLds wl;
    const int t = blockIdx.x, tid = threadIdx.x, K = H * AD;
    if (H == AH && tw_ok) {                                              // uniform: 8 heads, the row stays in registers (each
        float v[4];                                                      // lane holds 4 consecutive values) and is rotated and
        if (!combine_w_row(part, NC, T, causal, H, t, o, su, xs, wts, [] {}, v)) return;   // quantized on all 8 waves
        waves_rotate_quantize<8, 11>(v, wl, nullptr, nullptr, q8, scale, [] { __syncthreads(); }, t, q4, ldq);
        return;
    }
    if (!combine_w_row(part, NC, T, causal, H, t, o, su, xs, wts, [] {})) return;   // uniform
    // power-of-two rows (H = 1, 2, 4, 8) and 16-byte aligned INT8 outputs: the register + transpose engine on the first K / 16
    // threads (16 values each, read from the LDS row in layout 0); the same stages in the same order as the LDS engine, so
    // the same bits
    switch (tw_ok ? H : 0) {
        case 8: combine_rotate_quantize<11>(xs, red, q8, q4, ldq, scale, t); return;
        case 4: combine_rotate_quantize<10>(xs, red, q8, q4, ldq, scale, t); return;
        case 2: combine_rotate_quantize<9>(xs, red, q8, q4, ldq, scale, t); return;
        case 1: combine_rotate_quantize<8>(xs, red, q8, q4, ldq, scale, t); return;
        default: break;
    }
    float amx = 0.f;
    block_walsh(xs, K, [&](int i, float x) { xs[lds_slot(i)] = x; amx = fmaxf(amx, fabsf(x)); });
    const float sc = token_scale(block_max(amx, red));
    if (tid == 0) scale[t] = sc;
    quantize_row(xs, sc, q8 ? q8 + (size_t)t * K : nullptr, q4, t, K, ldq);
}

// grid M, H * 16 threads (H * AD = 1024 or 2048): thread 16 h + g owns dims 16 g .. 16 g + 15 of head h, summed over the
// chunks straight from the partials; the 16 lanes of head h first merge its chunk statistics (lane = chunk mod 16, a
// butterfly over the 16 lanes, so every lane holds the same total). With su, the BF16 row goes through the register Walsh
// engine and the quantizer of the output projection's prologue.
__global__ __launch_bounds__(128) void k_attn_combine_reg(const float* part, int NC, int T, int causal, int H, u16* o, const i8* su,
                                                          i8* q8, int* q4, int ldq, float* scale) {
    extern __shared__ float xs[];                                        // H * AD floats: cross-wave exchange
    __shared__ float wts[AH][MAXC];
    __shared__ float red[16];
    const int t = blockIdx.x, tid = threadIdx.x, h = tid >> 4, g = tid & 15, d0 = 16 * g, K = H * AD;
    const size_t cs = (size_t)H * PS;
    const float* hb = part + (size_t)t * NC * cs + (size_t)h * PS;      // head h of chunk 0
    const int NV = visible_chunks(NC, T, causal, t);
    // every load issued at entry: this lane's chunk statistics (chunks g, g + 16, ...) and the first 8 chunks' values
    constexpr int SC = MAXC / 16, VB = 8;
    typedef float f2_t __attribute__((ext_vector_type(2)));
    f2_t ml[SC];
#pragma unroll
    for (int r = 0; r < SC; ++r) {
        const int c = g + 16 * r;
        ml[r] = c < NV ? gptr((const f2_t*)(hb + c * cs + AD))[0] : f2_t{-__builtin_inff(), 0.f};
    }
    float4_t v0[VB][4];
#pragma unroll
    for (int i = 0; i < VB; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) v0[i][q] = i < NV ? gptr((const float4_t*)(hb + i * cs + d0))[q] : float4_t{0.f, 0.f, 0.f, 0.f};
    float mx = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < SC; ++r) mx = fmaxf(mx, ml[r].x);
    mx = row16_max(mx);
    float L = 0.f;
#pragma unroll
    for (int r = 0; r < SC; ++r) {
        const int c = g + 16 * r;
        if (c < NV) {
            const float w = ml[r].x == -__builtin_inff() ? 0.f : expf(ml[r].x - mx);
            wts[h][c] = w;                                               // read back by this wave only: LDS keeps its order
            L = __builtin_fmaf(w, ml[r].y, L);
        }
    }
    L = row16_sum(L);
    float acc[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) acc[k] = 0.f;
#pragma unroll
    for (int i = 0; i < VB; ++i) {
        if (i >= NV) break;
        const float w = wts[h][i];
#pragma unroll
        for (int k = 0; k < 16; ++k) acc[k] = __builtin_fmaf(w, v0[i][k >> 2][k & 3], acc[k]);
    }
    for (int c0 = VB; c0 < NV; c0 += 4) {
        float4_t v[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                v[i][q] = c0 + i < NV ? gptr((const float4_t*)(hb + (c0 + i) * cs + d0))[q] : float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (c0 + i >= NV) break;
            const float w = wts[h][c0 + i];
#pragma unroll
            for (int k = 0; k < 16; ++k) acc[k] = __builtin_fmaf(w, v[i][k >> 2][k & 3], acc[k]);
        }
    }
    u16 b[16];
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        b[k] = f32_to_bf16(acc[k] / L);
        v[k] = bf16_to_f32(b[k]);
    }
    if (o) {
        uint4_t w2[2];
#pragma unroll
        for (int k = 0; k < 8; ++k) w2[k >> 2][k & 3] = (u32)b[2 * k] | ((u32)b[2 * k + 1] << 16);
        u16* op = o + (size_t)t * K + h * AD + d0;
        gptr((uint4_t*)op)[0] = w2[0];
        gptr((uint4_t*)op)[1] = w2[1];
    }
    if (!su) return;
    const uint4_t sg = gptr((const uint4_t*)(su + h * AD + d0))[0];
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = v[k] * (float)(i8)(sg[k >> 2] >> (8 * (k & 3)));
    reg_rotate_quantize(v, K, xs, red, q8, q4, ldq, scale, t);
}

extern "C" int tcq_attend_chunks(int P, int M) { return (P + M + KC - 1) / KC; }

extern "C" int tcq_attend_q4(const void* q, const void* k_cache, const void* v_cache, int P, const void* k_new, const void* v_new,
                             int M, int H, int D, int causal_offset, float* part, void* o, const int8_t* su, int8_t* q8, int32_t* q4,
                             int ldq, float* scale, tcq_stream_t stream) {
    if (!q || !k_new || !v_new || !part || M <= 0 || H <= 0 || P < 0 || (P > 0 && (!k_cache || !v_cache))) return TCQ_ERR_ARG;
    if (!o && !su) return TCQ_ERR_ARG;
    if (su && ((!q8 && !q4) || !scale)) return TCQ_ERR_ARG;
    if (q4 && ldq != TCQ_LDQ_TOKEN_BLOCKS && ldq < M) return TCQ_ERR_ARG;
    if (q4 && ldq == TCQ_LDQ_TOKEN_BLOCKS && (uintptr_t)q4 % 16) return TCQ_ERR_ALIGN;
    if (D != AD || H > AH) return TCQ_ERR_UNSUPPORTED;
    if ((uintptr_t)k_new % 16 || (uintptr_t)k_cache % 16 || (uintptr_t)v_new % 16 || (uintptr_t)v_cache % 16 || (uintptr_t)part % 16)
        return TCQ_ERR_ALIGN;
    const int NC = tcq_attend_chunks(P, M);
    if (NC > MAXC) return TCQ_ERR_UNSUPPORTED;
    hipStream_t st = (hipStream_t)stream;
    // token pairs (16 MFMA rows): measured on MI355X at 50 tokens x 850 keys, 2 tokens per group run 12.5 us, 4 run 13.6 us
    // and 8 run 20 us (fewer, longer groups); single tokens (8 rows, half the MFMA rows empty) match pairs
    launch_k(k_attn_part<2>, dim3((M + 1) / 2, NC), dim3(AT), 0, st, (const u16*)q, (const u16*)k_cache, (const u16*)v_cache, P,
             (const u16*)k_new, (const u16*)v_new, M, H, causal_offset, part, AttnPost{});
    // combine: one wave per head with every load at entry (8-byte aligned o, 4-byte aligned su), else the register path for
    // H * AD of 1024 / 2048 (16-byte aligned outputs), else 1024 threads over LDS
    const bool oal = (!o || (uintptr_t)o % 16 == 0) && (!su || ((uintptr_t)su % 16 == 0 && (uintptr_t)q8 % 16 == 0));
    if ((!o || (uintptr_t)o % 8 == 0) && (!su || (uintptr_t)su % 4 == 0))
        launch_k(k_attn_combine_w, dim3(M), dim3(H * 64), su ? (size_t)lds_words(H * AD) * sizeof(float) : 0, st, (const float*)part,
                 NC, P + M, causal_offset, H, (u16*)o, (const i8*)su, (i8*)q8, (int*)q4, ldq, scale,
                 (int)((!q8 || (uintptr_t)q8 % 16 == 0) && (!q4 || ldq != TCQ_LDQ_TOKEN_BLOCKS || (uintptr_t)q4 % 16 == 0)));
    else if ((H == 4 || H == 8) && oal)
        launch_k(k_attn_combine_reg, dim3(M), dim3(H * 16), su ? (size_t)H * AD * sizeof(float) : 0, st, (const float*)part, NC,
                 P + M, causal_offset, H, (u16*)o, (const i8*)su, (i8*)q8, (int*)q4, ldq, scale);
    else
        launch_k(k_attn_combine, dim3(M), dim3(CT), su ? (size_t)lds_words(H * AD) * sizeof(float) : 0, st, (const float*)part, NC,
                 P + M, causal_offset, H, (u16*)o, (const i8*)su, (i8*)q8, (int*)q4, ldq, scale);
    return launch_status();
}

extern "C" int tcq_attend_parts(const void* q, const void* k_cache, const void* v_cache, int P, const void* k_new, const void* v_new,
                                int M, int H, int D, int causal_offset, float* part, tcq_stream_t stream) {
    if (!q || !k_new || !v_new || !part || M <= 0 || H <= 0 || P < 0 || (P > 0 && (!k_cache || !v_cache))) return TCQ_ERR_ARG;
    if (D != AD || H > AH) return TCQ_ERR_UNSUPPORTED;
    if ((uintptr_t)k_new % 16 || (uintptr_t)k_cache % 16 || (uintptr_t)v_new % 16 || (uintptr_t)v_cache % 16 || (uintptr_t)part % 16)
        return TCQ_ERR_ALIGN;
    const int NC = tcq_attend_chunks(P, M);
    if (NC > MAXC) return TCQ_ERR_UNSUPPORTED;
    launch_k(k_attn_part<2>, dim3((M + 1) / 2, NC), dim3(AT), 0, (hipStream_t)stream, (const u16*)q, (const u16*)k_cache,
             (const u16*)v_cache, P, (const u16*)k_new, (const u16*)v_new, M, H, causal_offset, part, AttnPost{});
    return launch_status();
}

extern "C" int tcq_attend_post_parts(const float* z_q, const float* z_k, const float* z_v, const int8_t* sv_q, const int8_t* sv_k,
                                     const int8_t* sv_v, const void* k_cache, const void* v_cache, int P, void* k_out, void* v_out,
                                     int H, int D, int causal_offset, float* part, tcq_stream_t stream) {
    if (!z_q || !z_k || !z_v || !sv_q || !sv_k || !sv_v || !k_out || !v_out || !part || P < 0 || (P > 0 && (!k_cache || !v_cache)))
        return TCQ_ERR_ARG;
    if (D != AD || H != AH) return TCQ_ERR_UNSUPPORTED;
    if ((uintptr_t)z_q % 16 || (uintptr_t)z_k % 16 || (uintptr_t)z_v % 16 || (uintptr_t)sv_q % 8 || (uintptr_t)sv_k % 8 ||
        (uintptr_t)sv_v % 8 || (uintptr_t)k_out % 16 || (uintptr_t)v_out % 16 || (uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 16 ||
        (uintptr_t)part % 16)
        return TCQ_ERR_ALIGN;
    const int NC = tcq_attend_chunks(P, 1);
    if (NC > MAXC) return TCQ_ERR_UNSUPPORTED;
    const AttnPost ap = {z_q, z_k, z_v, (const i8*)sv_q, (const i8*)sv_k, (const i8*)sv_v, (u16*)k_out, (u16*)v_out};
    launch_k(k_attn_part<2, true>, dim3(1, NC), dim3(AT), 0, (hipStream_t)stream, (const u16*)nullptr, (const u16*)k_cache,
             (const u16*)v_cache, P, (const u16*)nullptr, (const u16*)nullptr, 1, H, causal_offset, part, ap);
    return launch_status();
}

extern "C" int tcq_attend(const void* q, const void* k_cache, const void* v_cache, int P, const void* k_new, const void* v_new, int M,
                          int H, int D, int causal_offset, float* part, void* o, const int8_t* su, int8_t* q8, float* scale,
                          tcq_stream_t stream) {
    return tcq_attend_q4(q, k_cache, v_cache, P, k_new, v_new, M, H, D, causal_offset, part, o, su, q8, nullptr, 0, scale, stream);
}

// ------------------------------------------------------------------------------------------- allocation-free variant
// tcq_attend_q4 with the workspace in a file-scope device array instead of a caller's buffer, for callers that cannot
// allocate. Every (token, chunk, head) slot the combine reads is written by k_attn_part of the same call first, so the
// array needs no clearing; calls that overlap on one device share it and race.
constexpr size_t ATTEND_SCRATCH_FLOATS = (size_t)1 << 21;          // 8 MiB per device
static __device__ __align__(256) float scratch[ATTEND_SCRATCH_FLOATS];

namespace {
constexpr int SCRATCH_DEVICES = 64;
std::mutex scratch_mu;
float* scratch_ptr[SCRATCH_DEVICES] = {};

// The device address of `scratch` on the current device (its own copy per device), looked up once per device. The first
// call on a device may come while the caller captures a graph: the lookup is no stream work, so this thread's capture
// mode is relaxed around it (and restored), which lets it run under any capture mode.
int scratch_on_current_device(float** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SCRATCH_DEVICES) return TCQ_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_ptr[dev]) {
        void* p = nullptr;
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        hipError_t e = hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) return (int)e;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        const hipError_t r = hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) return (int)e;
        if (r != hipSuccess) return (int)r;
        scratch_ptr[dev] = (float*)p;
    }
    *out = scratch_ptr[dev];
    return TCQ_OK;
}
}  // namespace

extern "C" size_t tcq_attend_static_floats(void) { return ATTEND_SCRATCH_FLOATS; }

extern "C" int tcq_attend_q4_static(const void* q, const void* k_cache, const void* v_cache, int P, const void* k_new,
                                    const void* v_new, int M, int H, int D, int causal_offset, void* o, const int8_t* su, int8_t* q8,
                                    int32_t* q4, int ldq, float* scale, tcq_stream_t stream) {
    if (M <= 0 || H <= 0 || P < 0) return TCQ_ERR_ARG;
    if (D != AD || H > AH) return TCQ_ERR_UNSUPPORTED;
    if ((size_t)M * tcq_attend_chunks(P, M) * H * PS > ATTEND_SCRATCH_FLOATS) return TCQ_ERR_UNSUPPORTED;
    float* part = nullptr;
    const int e = scratch_on_current_device(&part);
    if (e) return e;
    return tcq_attend_q4(q, k_cache, v_cache, P, k_new, v_new, M, H, D, causal_offset, part, o, su, q8, q4, ldq, scale, stream);
}
