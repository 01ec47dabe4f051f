// Attention of H query heads over one shared key / value head (multi-query, head dim 256), BF16 in and out, FP32
// arithmetic: the attention of the Gemma decoder layers whose projections run on the TCQ kernels. The keys are the cache
// rows followed by this call's own rows, so no concatenated copy is made.
//
// Split over the keys (64 per chunk): k_attn_part computes, for one query token and one key chunk, the scores of every
// head, their chunk maximum m, the exponentials e = exp(s - m), l = sum e and the unnormalised outputs o = sum e v; then
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

// grid (tokens M, chunks NC), AT threads. part: (M, NC, H, AD + 2) FP32: o[AD], m, l per head.
// Keys: each pass of 64 keys loads its rows with 16-byte loads (the next pass's are in flight while one is used). Values:
// blocks of 64 rows staged in LDS with 16-byte loads (the next block's loads in flight while one is used), then one thread
// per dim walks the block's keys in order.
__global__ __launch_bounds__(AT) void k_attn_part(const u16* q, const u16* kc, const u16* vc, int P, const u16* kn, const u16* vn,
                                                  int M, int H, int causal, float* part) {
    __shared__ float qs[AH][AD];
    __shared__ float ps[AH][KC + 1];
    __shared__ __attribute__((aligned(16))) u16 vs[64][AD];
    const int t = blockIdx.x, c = blockIdx.y, NC = gridDim.y, tid = threadIdx.x;
    const int T = P + M, j0 = c * KC;
    const int jend = min(T, causal >= 0 ? causal + t + 1 : T);        // keys j < jend are visible to this query
    const int nvis = max(0, min(KC, jend - j0));                        // visible keys of this chunk
    const float scl = 1.f / 16.f;                                       // 1 / sqrt(256), exact
    if (nvis > 0) {
        for (int i = tid; i < AH * AD; i += AT) {
            const int h = i / AD, d = i - h * AD;
            qs[h][d] = h < H ? bf16_to_f32(gptr(q)[(size_t)t * H * AD + h * AD + d]) : 0.f;
        }
    }
    __syncthreads();
    const int npass = (nvis + 63) >> 6;
    // scores: thread (key kk = tid / 4, part p = tid % 4: dims 32 b + 8 p + e), 8 heads, reduced over the 4 parts; the
    // 4 parts of a key read adjacent 32-byte pieces of the query rows (different LDS banks)
    {
        const int p = tid & 3;
        uint4_t w[2][8];
        auto fetch = [&](int pass, uint4_t(&dst)[8]) {
            const int j = j0 + pass * 64 + (tid >> 2);
            if (pass < npass && j < jend) {
                const u16* kr = key_row(kc, kn, P, j) + 8 * p;
#pragma unroll
                for (int b = 0; b < 8; ++b) dst[b] = gptr((const uint4_t*)(kr + 32 * b))[0];
            }
        };
        fetch(0, w[0]);
#pragma unroll
        for (int pass = 0; pass < KC / 64; ++pass) {
            const int kk = pass * 64 + (tid >> 2), j = j0 + kk;
            if (pass + 1 < KC / 64) fetch(pass + 1, w[(pass + 1) & 1]);
            float a[AH];
#pragma unroll
            for (int h = 0; h < AH; ++h) a[h] = 0.f;
            if (pass < npass && j < jend) {
#pragma unroll
                for (int b = 0; b < 8; ++b) {
                    float kv[8];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        kv[2 * e] = bf16_to_f32((u16)(w[pass & 1][b][e] & 0xffffu));
                        kv[2 * e + 1] = bf16_to_f32((u16)(w[pass & 1][b][e] >> 16));
                    }
#pragma unroll
                    for (int h = 0; h < AH; ++h)
#pragma unroll
                        for (int e = 0; e < 8; ++e) a[h] = __builtin_fmaf(qs[h][32 * b + 8 * p + e], kv[e], a[h]);
                }
            }
#pragma unroll
            for (int h = 0; h < AH; ++h) {
                a[h] = a[h] + __shfl_xor(a[h], 1, 64);
                a[h] = a[h] + __shfl_xor(a[h], 2, 64);
            }
            if (p == 0) {
#pragma unroll
                for (int h = 0; h < AH; ++h) ps[h][kk] = j < jend ? a[h] * scl : -__builtin_inff();
            }
        }
    }
    __syncthreads();
    // chunk softmax statistics: wave w takes heads 2w, 2w + 1; lane holds keys lane + 64 i
    {
        const int w = tid >> 6, lane = tid & 63;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int h = 2 * w + hh;
            float sv[KC / 64], m = -__builtin_inff();
#pragma unroll
            for (int i = 0; i < KC / 64; ++i) {
                sv[i] = ps[h][lane + 64 * i];
                m = fmaxf(m, sv[i]);
            }
            m = wave_max(m);
            float l = 0.f;
#pragma unroll
            for (int i = 0; i < KC / 64; ++i) {
                const float e = m == -__builtin_inff() ? 0.f : expf(sv[i] - m);
                ps[h][lane + 64 * i] = e;
                l = l + e;
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) l = l + __shfl_xor(l, o, 64);
            if (lane == 0 && h < H) {
                float* base = part + (((size_t)t * NC + c) * H + h) * (AD + 2);
                base[AD] = m;
                base[AD + 1] = l;
            }
        }
    }
    // unnormalised outputs: thread = dim d, 8 heads, keys of the chunk in order, values from the LDS stage
    {
        const int d = tid;
        float o[AH];
#pragma unroll
        for (int h = 0; h < AH; ++h) o[h] = 0.f;
        uint4_t v[8];                                              // this thread's 8 of the block's 2048 16-byte granules
        auto vfetch = [&](int blk) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int gi = u * AT + tid, row = gi >> 5, col = gi & 31, j = j0 + blk * 64 + row;
                v[u] = j < jend ? gptr((const uint4_t*)(key_row(vc, vn, P, j) + 8 * col))[0] : uint4_t{0, 0, 0, 0};
            }
        };
        if (npass > 0) vfetch(0);
        for (int blk = 0; blk < npass; ++blk) {
            __syncthreads();                                       // ps complete (first block) / previous block consumed
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int gi = u * AT + tid;
                *(uint4_t*)&vs[gi >> 5][8 * (gi & 31)] = v[u];
            }
            __syncthreads();
            if (blk + 1 < npass) vfetch(blk + 1);
            const int kend = min(64, nvis - blk * 64);
            for (int kk = 0; kk < kend; ++kk) {
                const float x = bf16_to_f32(vs[kk][d]);
#pragma unroll
                for (int h = 0; h < AH; ++h) o[h] = __builtin_fmaf(ps[h][blk * 64 + kk], x, o[h]);
            }
        }
        for (int h = 0; h < H; ++h) part[(((size_t)t * NC + c) * H + h) * (AD + 2) + d] = o[h];
    }
}

// grid M, block 256 (one thread per dim). o (M, H * AD) BF16 (or NULL); with su, the row also goes through the rotate +
// quantize prologue (q8 row-major (M, H * AD), scale (M,)). The chunk statistics of the token are staged in LDS first and
// the weights exp(m_c - max m) computed once per (chunk, head); each thread then sums its dim over the chunks, the loads
// of all chunks in flight together.
constexpr int MAXC = 256;        // most chunks a token may have in the combine (16384 keys)
__global__ __launch_bounds__(256) void k_attn_combine(const float* part, int NC, int H, u16* o, const i8* su, i8* q8, float* scale) {
    extern __shared__ float lds[];
    __shared__ float red[16];
    __shared__ float wts[AH][MAXC];
    __shared__ float ls[AH][MAXC];
    __shared__ float inv[AH];
    const int t = blockIdx.x, d = threadIdx.x, K = H * AD;
    const size_t cs = (size_t)H * (AD + 2);                          // stride between chunks
    const float* tb = part + (size_t)t * NC * cs;
    for (int i = threadIdx.x; i < H * NC; i += blockDim.x) {
        const int h = i / NC, c = i - h * NC;
        wts[h][c] = tb[c * cs + h * (AD + 2) + AD];                  // m
        ls[h][c] = tb[c * cs + h * (AD + 2) + AD + 1];               // l
    }
    __syncthreads();
    if (threadIdx.x < H) {
        const int h = threadIdx.x;
        float mx = -__builtin_inff();
        for (int c = 0; c < NC; ++c) mx = fmaxf(mx, wts[h][c]);
        float L = 0.f;
        for (int c = 0; c < NC; ++c) {
            const float m = wts[h][c];
            const float w = m == -__builtin_inff() ? 0.f : expf(m - mx);
            L = L + w * ls[h][c];
            wts[h][c] = w;
        }
        inv[h] = L;
    }
    __syncthreads();
    float acc[AH];
#pragma unroll
    for (int h = 0; h < AH; ++h) acc[h] = 0.f;
#pragma unroll 4
    for (int c = 0; c < NC; ++c) {
        const float* col = tb + c * cs + d;
        float v[AH];
#pragma unroll
        for (int h = 0; h < AH; ++h) v[h] = h < H ? col[h * (AD + 2)] : 0.f;
#pragma unroll
        for (int h = 0; h < AH; ++h) acc[h] = __builtin_fmaf(wts[h][c], v[h], acc[h]);
    }
    for (int h = 0; h < H; ++h) {
        const u16 b = f32_to_bf16(acc[h] / inv[h]);
        if (o) gptr(o)[(size_t)t * K + h * AD + d] = b;
        if (su) lds[lds_slot(h * AD + d)] = bf16_to_f32(b) * (float)gptr(su)[h * AD + d];
    }
    if (!su) return;
    __syncthreads();
    float amx = 0.f;
    block_walsh(lds, K, [&](int i, float v) { lds[lds_slot(i)] = v; amx = fmaxf(amx, fabsf(v)); });
    const float sc = token_scale(block_max(amx, red));
    if (threadIdx.x == 0) scale[t] = sc;
    quantize_row(lds, sc, q8 + (size_t)t * K, nullptr, t, K, 0);
}

// =========================================================================================================== C ABI
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
    launch_k(k_attn_combine, dim3(M), dim3(256), su ? (size_t)lds_words(H * AD) * sizeof(float) : 0, st, (const float*)part, NC, H,
             (u16*)o, (const i8*)su, (i8*)q8, scale);
    return launch_status();
}
