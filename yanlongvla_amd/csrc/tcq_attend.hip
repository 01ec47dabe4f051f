// Attention of H query heads over one shared key / value head (multi-query, head dim 256), BF16 in and out, FP32
// arithmetic: the attention of the Gemma decoder layers whose projections run on the TCQ kernels. The keys are the cache
// rows followed by this call's own rows, so no concatenated copy is made.
//
// Split over the keys (64 per chunk): k_attn_part computes, for one query token and one key chunk, the scores of every
// head (BF16 MFMA, FP32 sums), their chunk maximum m, the exponentials e = exp(s - m), l = sum e (FP32) and the unnormalised
// outputs o = sum bf16(e) v (BF16 MFMA, FP32 sums); then
// k_attn_combine merges the chunks of a token (weights exp(m_c - max_c m_c)) and divides by the merged sum. The result
// depends on the number of keys only through this fixed chunking, never on launch shapes. The combine can feed its BF16
// output row straight into the rotate + quantize prologue of the output projection. The dot products and weighted sums
// use fused multiply-adds (this attention is the decoder layers' own definition, not a reference rounding chain).
#include "tcq_device.h"
#include "tcq_launch.h"

namespace {

constexpr int AD = 256;          // head dim
constexpr int AH = 8;            // most query heads
constexpr int KC = 64;           // keys per chunk
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

// grid (tokens M, chunks NC), AT = 256 threads (4 waves). part: (M, NC, H, AD + 2) FP32: o[AD], m, l per head.
// Scores on v_mfma_f32_16x16x32_bf16: A = the query rows of the token (heads 0..7, rows 8..15 zero), B = 16 keys per wave, 8
// K steps of 32 dims; lane (g, c) of D holds heads 4g..4g+3 of key c. Softmax statistics per head over the chunk's 64 keys.
// Outputs on the same MFMA: A = the exponentials e (BF16, heads x keys), B = 16 value columns x 32 keys gathered from the LDS
// stage; each wave owns 4 of the 16 column tiles, 2 K steps. Element i of lane group lg in K step ks is key 32 ks + lg + 4 i
// in both operands (any common order of the K index gives the same product).
__global__ __launch_bounds__(AT) void k_attn_part(const u16* q, const u16* kc, const u16* vc, int P, const u16* kn, const u16* vn,
                                                  int M, int H, int causal, float* part) {
    __shared__ float ps[AH][KC + 1];
    __shared__ __attribute__((aligned(16))) u16 vs[KC][VST];
    const int t = blockIdx.x, c = blockIdx.y, NC = gridDim.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int T = P + M, j0 = c * KC;
    const int jend = min(T, causal >= 0 ? causal + t + 1 : T);        // keys j < jend are visible to this query
    const int nvis = max(0, min(KC, jend - j0));                        // visible keys of this chunk
    const float scl = 1.f / 16.f;                                       // 1 / sqrt(256), exact
    // value stage: 64 rows x 256 dims, 8 granules of 16 bytes per thread, issued first
    uint4_t vg[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int gi = u * AT + tid, row = gi >> 5, col = gi & 31, j = j0 + row;
        vg[u] = j < jend ? gptr((const uint4_t*)(key_row(vc, vn, P, j) + 8 * col))[0] : uint4_t{0, 0, 0, 0};
    }
    // scores
    {
        const int j = j0 + 16 * wave + lr;                               // this lane's key (B column)
        const bool kv = j < jend;
        const u16* kr = kv ? key_row(kc, kn, P, j) : nullptr;
        const u16* qr = q + (size_t)t * H * AD + (size_t)lr * AD;        // query row of head lr (A row)
        float4_t acc = {0.f, 0.f, 0.f, 0.f};
        uint4_t A[8], B[8];
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            A[ks] = lr < H ? gptr((const uint4_t*)(qr + 32 * ks + 8 * lg))[0] : uint4_t{0, 0, 0, 0};
            B[ks] = kv ? gptr((const uint4_t*)(kr + 32 * ks + 8 * lg))[0] : uint4_t{0, 0, 0, 0};
        }
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) acc = mma_bf16(A[ks], B[ks], acc);
        if (lg < 2) {
#pragma unroll
            for (int e = 0; e < 4; ++e) ps[4 * lg + e][16 * wave + lr] = kv ? acc[e] * scl : -__builtin_inff();
        }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int gi = u * AT + tid;
        *(uint4_t*)&vs[gi >> 5][8 * (gi & 31)] = vg[u];
    }
    __syncthreads();
    // chunk softmax statistics: wave w takes heads 2w, 2w + 1, lane = key
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const int h = 2 * wave + hh;
        const float sv = ps[h][lane];
        const float m = wave_max(sv);
        const float e = m == -__builtin_inff() ? 0.f : expf(sv - m);
        float l = e;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) l = l + __shfl_xor(l, o, 64);
        ps[h][lane] = e;
        if (lane == 0 && h < H) {
            float* base = part + (((size_t)t * NC + c) * H + h) * (AD + 2);
            base[AD] = m;
            base[AD + 1] = l;
        }
    }
    __syncthreads();
    // unnormalised outputs o[h][d] = sum_k e[h][k] v[k][d]
    {
        uint4_t A[2];                                                   // e of heads lr (< 8), BF16
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            u32 w[4];
#pragma unroll
            for (int k2 = 0; k2 < 4; ++k2) {
                const int k0 = 32 * ks + lg + 8 * k2;                   // elements 2 k2, 2 k2 + 1: keys k0, k0 + 4
                const float e0 = lr < AH ? ps[lr][k0] : 0.f, e1 = lr < AH ? ps[lr][k0 + 4] : 0.f;
                w[k2] = (u32)f32_to_bf16(e0) | ((u32)f32_to_bf16(e1) << 16);
            }
            A[ks] = uint4_t{w[0], w[1], w[2], w[3]};
        }
#pragma unroll
        for (int tl = 0; tl < 4; ++tl) {
            const int d = 16 * (4 * wave + tl) + lr;                     // this lane's value column
            float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                u32 w[4];
#pragma unroll
                for (int k2 = 0; k2 < 4; ++k2) {
                    const int k0 = 32 * ks + lg + 8 * k2;
                    w[k2] = (u32)vs[k0][d] | ((u32)vs[k0 + 4][d] << 16);
                }
                acc = mma_bf16(A[ks], uint4_t{w[0], w[1], w[2], w[3]}, acc);
            }
            if (lg < 2) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int h = 4 * lg + e;
                    if (h < H) part[(((size_t)t * NC + c) * H + h) * (AD + 2) + d] = acc[e];
                }
            }
        }
    }
}

// grid M, CT = 1024 threads: thread (d, g) = (tid % 256, tid / 256) sums dim d of every head over the chunks c = g (mod 4);
// wave h < H first merges head h's chunk statistics (lane = chunk). The four partial sums of a head add in the fixed order
// ((g0 + g1) + g2) + g3, so the result depends only on NC. With su set, the BF16 row (H x 256) is rotated and quantized
// in place as the output projection's prologue.
constexpr int MAXC = 256;        // most chunks a token may have in the combine (16384 keys)
constexpr int CT = 1024, CG = CT / AD, CB = 4;   // threads, chunk groups, chunks per group held in registers per batch

__global__ __launch_bounds__(CT) void k_attn_combine(const float* part, int NC, int H, u16* o, const i8* su, i8* q8, float* scale) {
    extern __shared__ float lds[];
    __shared__ float red[CT / 64];
    __shared__ float wts[AH][MAXC];
    __shared__ float inv[AH];
    __shared__ float sums[CG][AH][AD];
    const int t = blockIdx.x, tid = threadIdx.x, d = tid & (AD - 1), g = tid / AD, lane = tid & 63, wave = tid >> 6, K = H * AD;
    const size_t cs = (size_t)H * (AD + 2);                          // stride between chunks
    const float* tb = part + (size_t)t * NC * cs;
    constexpr int SR = MAXC / 64;
    float mv[SR], lv[SR];
    if (wave < H) {
#pragma unroll
        for (int r = 0; r < SR; ++r) {
            const int c = 64 * r + lane;
            mv[r] = c < NC ? tb[c * cs + wave * (AD + 2) + AD] : -__builtin_inff();
            lv[r] = c < NC ? tb[c * cs + wave * (AD + 2) + AD + 1] : 0.f;
        }
    }
    float v[CB][AH];
    auto load = [&](int c0) {
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int c = c0 + g + CG * i;
#pragma unroll
            for (int h = 0; h < AH; ++h) v[i][h] = c < NC && h < H ? tb[c * cs + h * (AD + 2) + d] : 0.f;
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
            if (c < NC) wts[wave][c] = w;
            L = __builtin_fmaf(w, lv[r], L);
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) L = L + __shfl_xor(L, off, 64);
        if (lane == 0) inv[wave] = L;
    }
    __syncthreads();
    float acc[AH];
#pragma unroll
    for (int h = 0; h < AH; ++h) acc[h] = 0.f;
    for (int c0 = 0; c0 < NC; c0 += CG * CB) {
        if (c0) load(c0);
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int c = c0 + g + CG * i;
            if (c < NC) {
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
    quantize_row(lds, sc, q8 + (size_t)t * K, nullptr, t, K, 0);
}

extern "C" int tcq_attend_chunks(int P, int M) { return (P + M + KC - 1) / KC; }

extern "C" int tcq_attend(const void* q, const void* k_cache, const void* v_cache, int P, const void* k_new, const void* v_new, int M,
                          int H, int D, int causal_offset, float* part, void* o, const int8_t* su, int8_t* q8, float* scale,
                          tcq_stream_t stream) {
    if (!q || !k_new || !v_new || !part || M <= 0 || H <= 0 || P < 0 || (P > 0 && (!k_cache || !v_cache))) return TCQ_ERR_ARG;
    if (!o && !su) return TCQ_ERR_ARG;
    if (su && (!q8 || !scale)) return TCQ_ERR_ARG;
    if (D != AD || H > AH) return TCQ_ERR_UNSUPPORTED;
    if ((uintptr_t)k_new % 16 || (uintptr_t)k_cache % 16 || (uintptr_t)v_new % 16 || (uintptr_t)v_cache % 16) return TCQ_ERR_ALIGN;
    const int NC = tcq_attend_chunks(P, M);
    if (NC > MAXC) return TCQ_ERR_UNSUPPORTED;
    hipStream_t st = (hipStream_t)stream;
    launch_k(k_attn_part, dim3(M, NC), dim3(AT), 0, st, (const u16*)q, (const u16*)k_cache, (const u16*)v_cache, P,
             (const u16*)k_new, (const u16*)v_new, M, H, causal_offset, part);
    launch_k(k_attn_combine, dim3(M), dim3(CT), su ? (size_t)lds_words(H * AD) * sizeof(float) : 0, st, (const float*)part, NC, H,
             (u16*)o, (const i8*)su, (i8*)q8, scale);
    return launch_status();
}
