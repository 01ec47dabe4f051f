// Small-M INT8 products (M <= 64 tokens) on v_mfma_i32_16x16x64_i8: the W2A8 fused trellis decode + product, and the same
// product on resident INT8 weights. z[t, i] = (float(acc[t, i]) * s[t]) * rs[i], acc exact in int32 (the reference's
// finish(), deploy/tcq_kernels/kernels.py:355-363).
//
// MFMA mapping per 256-column chunk c and j = 0..3: A = weights, lane (g, r) = row r of the tile row, k-block g = the 16
// columns of tile 16 c + 4 j + g (exactly one decoded tile row per lane); B = activations, lane (g, t) = token t of the
// token block, the same 16 columns; D: lane (g, t) holds rows 4 g .. 4 g + 3 of token t.
// A from the trellis words: the window layout of tcq_repack (one dwordx4 per lane per tile row and chunk), 8 lookups of
// INT8 pairs in a sign-folded LDS table (1024 entries x 16 copies, one 4-byte slot each, lane l reads copy l mod 16), packed
// into the 16 A bytes. A from resident INT8 weights: one 16-byte load per lane per (tile row, j).
// The activations of a chunk (16 NB tokens x 256 bytes, zero for tokens >= M and columns >= K) are staged in LDS, double
// buffered, with an XOR swizzle of the 16-byte granules by token so that the 16 tokens of a B read hit different banks.
#include "tcq_device.h"
#include "tcq_launch.h"

namespace {

constexpr int SM_C = 16;               // table copies
constexpr int SM_THREADS = 512;

typedef int int4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void fill_table_i8(u32* tab, const i8* t8) {
    for (int e = threadIdx.x; e < 1024; e += blockDim.x) {
        const int h = e & 511;
        int v0 = gptr(t8)[2 * h];
        const int v1 = gptr(t8)[2 * h + 1];
        if (e >> 9) v0 = -v0;
        const u32 v = (u32)(v0 & 0xff) | ((u32)(v1 & 0xff) << 8);
        const u32 vv = v | (v << 16);
#pragma unroll
        for (int c = 0; c < SM_C; c += 4) *(uint4_t*)(tab + e * SM_C + c) = uint4_t{vv, vv, vv, vv};
    }
}

// stage the activations of chunk c: buffer (16 NB tokens) x 256 bytes, granule (t, g16) at t * 256 + 16 * (g16 ^ (t & 15))
template <int NB>
__device__ __forceinline__ void stage_load(const i8* q, int M, int K, int c, uint4_t (&v)[NB / 2 > 0 ? NB / 2 : 1]) {
    constexpr int G = NB * 16 * 16, PER = (G + SM_THREADS - 1) / SM_THREADS;
    static_assert(PER <= (NB / 2 > 0 ? NB / 2 : 1), "staging registers");
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int gi = threadIdx.x + p * SM_THREADS;
        const int t = gi >> 4, k = 256 * c + 16 * (gi & 15);
        v[p] = (gi < G && t < M && k < K) ? gptr((const uint4_t*)(q + (size_t)t * K + k))[0] : uint4_t{0, 0, 0, 0};
    }
}
template <int NB>
__device__ __forceinline__ void stage_store(char* buf, const uint4_t (&v)[NB / 2 > 0 ? NB / 2 : 1]) {
    constexpr int G = NB * 16 * 16, PER = (G + SM_THREADS - 1) / SM_THREADS;
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int gi = threadIdx.x + p * SM_THREADS;
        if (gi < G) {
            const int t = gi >> 4, g16 = gi & 15;
            *(uint4_t*)(buf + t * 256 + 16 * (g16 ^ (t & 15))) = v[p];
        }
    }
}

}  // namespace

// grid (workgroups per segment, segments). A workgroup covers 8 R tile rows of its segment (wave w: rows w R .. w R + R - 1)
// for all chunks; the words / weights of chunk c + 1 and the activations of chunk c + 1 are loaded while chunk c is
// multiplied. MODE 0: decode from tcq_repack words; MODE 1: resident INT8 weights.
template <int MODE, int NB, int R>
__global__ __launch_bounds__(SM_THREADS) void k_gemm_small(const tcq_gemm_seg* segs, const i8* q, const float* s, int M, int K,
                                                          int ldz) {
    __shared__ __attribute__((aligned(16))) u32 tab[MODE == 0 ? 1024 * SM_C : 4];
    __shared__ __attribute__((aligned(16))) char bq[2][NB * 16 * 256];
    const tcq_gemm_seg S = segs[blockIdx.y];
    const int tiles_m = S.m >> 4, nch = (K + 255) >> 8;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int lr = lane & 15, lg = lane >> 4;
    const int I0 = (blockIdx.x * (SM_THREADS / 64) + wave) * R;           // first tile row of this wave
    if (blockIdx.x * (SM_THREADS / 64) * R >= tiles_m) return;           // whole workgroup past the segment (uniform)
    if (MODE == 0) fill_table_i8(tab, S.t8);

    uint4_t st[NB / 2 > 0 ? NB / 2 : 1];
    stage_load<NB>(q, M, K, 0, st);
    stage_store<NB>(bq[0], st);
    const bool active = I0 < tiles_m;
    const int lastI = tiles_m - 1;
    const u32 cp4 = (u32)(lane & (SM_C - 1)) << 2;

    // A sources
    uint4_t wa[2][R][MODE == 0 ? 1 : 4];
    rsrc_t Wr;
    if (MODE == 0) Wr = make_rsrc(S.w, (u32)(tiles_m * nch) << 10);
    else Wr = make_rsrc(S.w, (u32)S.m * (u32)K);
    auto loadA = [&](uint4_t(&dst)[R][MODE == 0 ? 1 : 4], int c) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int I = min(I0 + r, lastI);
            if (MODE == 0) {
                dst[r][0] = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(Wr, (u32)lane << 4,
                                                                                              (u32)(I * nch + c) << 10, 2));
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int k0 = 256 * c + 64 * j + 16 * lg;
                    const u32 off = (u32)(16 * I + lr) * (u32)K + (u32)k0;
                    dst[r][j] = k0 < K ? __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(Wr, off, 0, 2))
                                       : uint4_t{0, 0, 0, 0};
                }
            }
        }
    };

    int4v acc[R][NB];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[r][b] = int4v{0, 0, 0, 0};

    if (active) loadA(wa[0], 0);
    __syncthreads();

    for (int c = 0; c < nch; ++c) {
        const int cur = c & 1;
        if (c + 1 < nch) stage_load<NB>(q, M, K, c + 1, st);
        if (active && c + 1 < nch) loadA(wa[cur ^ 1], c + 1);
        if (active) {
            const char* bb = bq[cur];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                int4v B[NB];
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const int t = 16 * b + lr;
                    B[b] = *(const int4v*)(bb + t * 256 + 16 * ((4 * j + lg) ^ (t & 15)));
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    int4v A;
                    if (MODE == 0) {
                        const u32 hi = wa[cur][r][0][j];
                        const u32 hn = (u32)__builtin_amdgcn_mov_dpp((int)hi, 0x12F, 0xf, 0xf, false);
                        u32 e0[4], e1[4];
#pragma unroll
                        for (int p = 0; p < 4; ++p) {
                            const u32 x = pk_code(p == 0 ? hi : __builtin_amdgcn_alignbit(hi, hn, 32 - 4 * p));
                            e0[p] = *(const u16*)((const char*)tab + (((x >> 22) << 6) | cp4));           // pair p
                            e1[p] = *(const u16*)((const char*)tab + (((x >> 6) & 1023u) << 6 | cp4));     // pair p + 4
                        }
                        A = int4v{(int)(e0[0] | (e0[1] << 16)), (int)(e0[2] | (e0[3] << 16)), (int)(e1[0] | (e1[1] << 16)),
                                  (int)(e1[2] | (e1[3] << 16))};
                    } else {
                        A = __builtin_bit_cast(int4v, wa[cur][r][j]);
                    }
#pragma unroll
                    for (int b = 0; b < NB; ++b) acc[r][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B[b], acc[r][b], 0, 0, 0);
                }
            }
        }
        if (c + 1 < nch) stage_store<NB>(bq[cur ^ 1], st);
        __syncthreads();
    }
    if (!active) return;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int I = I0 + r;
        if (I >= tiles_m) continue;
        const float4_t rsv = gptr((const float4_t*)(S.rs + 16 * I + 4 * lg))[0];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int t = 16 * b + lr;
            if (t < M) {
                const float st_ = gptr(s)[t];
                float4_t o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = ((float)acc[r][b][e] * st_) * rsv[e];
                *gptr((float4_t*)(S.z + (size_t)t * ldz + 16 * I + 4 * lg)) = o;
            }
        }
    }
}

// =========================================================================================================== C ABI
template <int MODE>
static int gemm_small(const tcq_gemm_seg* segs, int nseg, int max_m, const int8_t* q, const float* s, int M, int K, int ldz,
                      tcq_stream_t stream) {
    if (!segs || !q || !s || nseg <= 0 || max_m <= 0 || M <= 0 || K <= 0 || ldz <= 0) return TCQ_ERR_ARG;
    if (max_m % 16 || K % 16) return TCQ_ERR_SHAPE;
    if (M > 64 || nseg > 65535) return TCQ_ERR_UNSUPPORTED;
    if ((uintptr_t)q % 16 || ldz % 4) return TCQ_ERR_ALIGN;
    if ((size_t)max_m * K >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
    constexpr int R = 2, WROWS = (SM_THREADS / 64) * R;
    const dim3 grid((max_m / 16 + WROWS - 1) / WROWS, nseg), block(SM_THREADS);
    hipStream_t st = (hipStream_t)stream;
    const i8* qq = (const i8*)q;
    if (M <= 16) launch_k(k_gemm_small<MODE, 1, R>, grid, block, 0, st, segs, qq, s, M, K, ldz);
    else if (M <= 32) launch_k(k_gemm_small<MODE, 2, R>, grid, block, 0, st, segs, qq, s, M, K, ldz);
    else launch_k(k_gemm_small<MODE, 4, R>, grid, block, 0, st, segs, qq, s, M, K, ldz);
    return launch_status();
}

extern "C" int tcq_gemm_tcq(const tcq_gemm_seg* segs, int nseg, int max_m, const int8_t* q, const float* s, int M, int K, int ldz,
                            tcq_stream_t stream) {
    return gemm_small<0>(segs, nseg, max_m, q, s, M, K, ldz, stream);
}

extern "C" int tcq_gemm_w8(const tcq_gemm_seg* segs, int nseg, int max_m, const int8_t* q, const float* s, int M, int K, int ldz,
                           tcq_stream_t stream) {
    return gemm_small<1>(segs, nseg, max_m, q, s, M, K, ldz, stream);
}
