// W2 float path products (BF16 rotated activations, the INT8 table values as weights, FP32 sums) on
// v_mfma_f32_16x16x32_bf16: the fused trellis decode + product and the same product on resident INT8 weights. The
// reference's k_gemmf_tcq / k_gemmf_w8 (deploy/tcq_kernels/kernels.py:430-489) compute z[t, i] = (sum_k w[i, k] h[t, k]) *
// rs[i] in FP32; here the sum runs in MFMA blocks, so its rounding differs from the reference's lane-sequential sums in the
// last bits (the layer is defined within 2e-3 of the FP64 sums).
//
// MFMA mapping per 256-column chunk c and j = 0..3 (one 16 x 16 tile per lane group, as the INT8 small-M products):
// A = weights, lane (g, r) = row r of the tile row, weights 0..7 (A0) and 8..15 (A1) of tile 16 c + 4 j + g;
// B = activations, lane (g, t) = token t of the token block, columns 256 c + 64 j + 16 g + 0..7 (B0) and + 8..15 (B1);
// D: lane (g, t) holds rows 4 g .. 4 g + 3 of token t.
// A from the trellis words: 8 lookups of BF16 pairs in a sign-folded LDS table (1024 entries x FC copies, one 4-byte slot
// each: entry e = (bf16(t8[e & 511][0]) with its sign bit flipped when e >> 9, bf16(t8[e & 511][1])), the reference's BF16
// images of the INT8 table, kernels.py:319-337), the two MFMA operands straight from the gathers. A from resident INT8
// weights: one 16-byte load per lane per (tile row, j), each byte converted to BF16 (exact: |w| <= 127).
// Work split: a workgroup takes one tile row of one segment and one group of 16 NB tokens (grid.z), its waves split K, one
// 256-column chunk each (wave w takes chunks w, w + NW, ...); the waves' FP32 partial sums meet in LDS in wave order.
#include "tcq_device.h"
#include "tcq_launch.h"

namespace {

constexpr int FC = 4;                  // table copies (lane l reads copy l mod FC)

typedef int int4v __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

struct FSegPack {
    tcq_gemm_seg s[TCQ_MAX_SEGS];
};

enum { HL_ROWS = 0, HL_COLS = 1 };     // activations h (M, K) row-major, or hT (K, ldh) with token = column

__device__ __forceinline__ void fill_table_bf16(u32* tab, const i8* t8) {
    for (int e = threadIdx.x; e < 1024; e += blockDim.x) {
        const int h = e & 511;
        const u32 b0 = (__float_as_uint((float)gptr(t8)[2 * h]) >> 16) ^ ((u32)(e >> 9) << 15);
        const u32 b1 = __float_as_uint((float)gptr(t8)[2 * h + 1]) & 0xffff0000u;
        const u32 v = b0 | b1;
        *(uint4_t*)(tab + e * FC) = uint4_t{v, v, v, v};
    }
}

// four INT8 weights of one dword -> two words of two BF16 (weight 0 in the low half of lo)
__device__ __forceinline__ void i8x4_to_bf16(u32 w, u32& lo, u32& hi) {
    const float f0 = (float)(i8)w, f1 = (float)(i8)(w >> 8), f2 = (float)(i8)(w >> 16), f3 = (float)(i8)(w >> 24);
    lo = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
    hi = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
}

__device__ __forceinline__ float4_t mma_bf16(int4v a, int4v b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

}  // namespace

// grid (tile rows of the largest segment, segments, token groups of 16 NB); NW = blockDim.x / 64 <= FMAXW waves.
// MODE 0: decode from tcq_repack words (RB: the reference's stored word layout, 64 bytes per tile, tiles row-major);
// MODE 1: resident INT8 weights (m, K). ODT F32: z = acc * rs; BF16: bf16(acc), unscaled (the prefill product's rounding,
// scaled by rs in its epilogue). HL: activation layout (ldh only for HL_COLS).
// waves per workgroup at most: 16 for one token block from row-major activations, else 8 (512 threads, 256 registers:
// the activation fragments of 2 or 4 token blocks, or the 16 gathered columns of hT, do not fit 128)
template <int NB, int HL> struct FWaves { static constexpr int max = NB == 1 && HL == HL_ROWS ? 16 : 8; };

template <int MODE, int NB, int ODT, int HL, bool RB>
__global__ __launch_bounds__((64 * FWaves<NB, HL>::max)) void k_gemmf_small(const FSegPack P, const u16* h, int M, int K, int ldh, int ldz) {
    constexpr int MAXW = FWaves<NB, HL>::max;
    __shared__ __attribute__((aligned(16))) u32 tab[MODE == 0 ? 1024 * FC : 4];
    __shared__ __attribute__((aligned(16))) float4_t red[(MAXW - 1) * NB * 64];
    const tcq_gemm_seg S = P.s[blockIdx.y];
    const int tiles_m = S.m >> 4, nch = (K + 255) >> 8, tiles_n = K >> 4;
    const int I = blockIdx.x;
    if (I >= tiles_m) return;                                             // uniform
    const int t0 = (int)blockIdx.z * 16 * NB;
    const int nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int lr = lane & 15, lg = lane >> 4;
    const u32 cp4 = (u32)(lane & (FC - 1)) << 2;
    rsrc_t Wr;
    if (MODE == 0) Wr = make_rsrc(S.w, RB ? (u32)(tiles_m * tiles_n) << 6 : (u32)(tiles_m * nch) << 10);
    else Wr = make_rsrc(S.w, (u32)S.m * (u32)K);
    const rsrc_t H = make_rsrc(h, HL == HL_ROWS ? (u32)M * (u32)K * 2u : (u32)K * (u32)ldh * 2u);

    uint4_t wa[MODE == 0 ? 1 : 4];
    int4v B[4][NB][2];
    auto load = [&](int c) {                                              // weights / words and activations of chunk c
        if (MODE == 0 && RB) {                                            // dword lr of tile 16 c + 4 j + lg, halves swapped
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int J = 16 * c + 4 * j + lg;
                const u32 off = J < tiles_n ? (((u32)(I * tiles_n + J) << 6) | ((u32)lr << 2)) : RSRC_OOB;
                const u32 d = __builtin_amdgcn_raw_buffer_load_b32(Wr, off, 0, 2);
                wa[0][j] = __builtin_amdgcn_alignbit(d, d, 16);
            }
        } else if (MODE == 0) {
            wa[0] = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(Wr, (u32)lane << 4, (u32)(I * nch + c) << 10, 2));
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k0 = 256 * c + 64 * j + 16 * lg;
                const u32 off = k0 < K ? (u32)(16 * I + lr) * (u32)K + (u32)k0 : RSRC_OOB;
                wa[j] = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(Wr, off, 0, 2));
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int t = t0 + 16 * b + lr, k = 256 * c + 64 * j + 16 * lg;
                const bool in = t < M && k < K;                           // K % 16 == 0: a fragment is all in or all out
                if (HL == HL_ROWS) {
                    const u32 off = (u32)t * (u32)K + (u32)k;
                    B[j][b][0] = __builtin_bit_cast(int4v, __builtin_amdgcn_raw_buffer_load_b128(H, in ? off * 2u : RSRC_OOB, 0, 0));
                    B[j][b][1] = __builtin_bit_cast(int4v, __builtin_amdgcn_raw_buffer_load_b128(H, in ? off * 2u + 16u : RSRC_OOB, 0, 0));
                } else {                                                  // 16 columns of token t: 16 elements ldh apart
                    u32 e[16];
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        e[i] = __builtin_amdgcn_raw_buffer_load_b16(H, in ? ((u32)(k + i) * (u32)ldh + (u32)t) * 2u : RSRC_OOB, 0, 0);
#pragma unroll
                    for (int i = 0; i < 8; ++i) B[j][b][i >> 2][i & 3] = (int)(e[2 * i] | (e[2 * i + 1] << 16));
                }
            }
    };

    float4_t acc[NB][2];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b][0] = acc[b][1] = float4_t{0.f, 0.f, 0.f, 0.f};
    if (wave < nch) load(wave);
    float4_t rsv = float4_t{0.f, 0.f, 0.f, 0.f};
    if (ODT == TCQ_F32 && wave == 0) rsv = gptr((const float4_t*)(S.rs + 16 * I + 4 * lg))[0];
    if (MODE == 0) fill_table_bf16(tab, S.t8 + (S.rows_per_table > 0 ? (size_t)(16 * I / S.rows_per_table) * 1024 : 0));
    __syncthreads();
    for (int c = wave; c < nch; c += nw) {
        if (c != wave) load(c);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int4v A0, A1;
            if (MODE == 0) {
                const u32 hi = wa[0][j];
                const u32 hn = (u32)__builtin_amdgcn_mov_dpp((int)hi, 0x12F, 0xf, 0xf, false);
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const u32 x = pk_code(p == 0 ? hi : __builtin_amdgcn_alignbit(hi, hn, 32 - 4 * p));
                    A0[p] = *(const int*)((const char*)tab + (((x >> 22) << 4) | cp4));             // pair p
                    A1[p] = *(const int*)((const char*)tab + ((((x >> 6) & 1023u) << 4) | cp4));    // pair p + 4
                }
            } else {
                u32 v[8];
#pragma unroll
                for (int d = 0; d < 4; ++d) i8x4_to_bf16(wa[j][d], v[2 * d], v[2 * d + 1]);
                A0 = int4v{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
                A1 = int4v{(int)v[4], (int)v[5], (int)v[6], (int)v[7]};
            }
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                acc[b][0] = mma_bf16(A0, B[j][b][0], acc[b][0]);
                acc[b][1] = mma_bf16(A1, B[j][b][1], acc[b][1]);
            }
        }
    }
    // sum the waves' partial FP32 sums through LDS in wave order, then scale and store
    if (wave > 0) {
#pragma unroll
        for (int b = 0; b < NB; ++b) red[((wave - 1) * NB + b) * 64 + lane] = acc[b][0] + acc[b][1];
    }
    __syncthreads();
    if (wave != 0) return;
    float4_t a[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) a[b] = acc[b][0] + acc[b][1];
    for (int w = 0; w < nw - 1; ++w)
#pragma unroll
        for (int b = 0; b < NB; ++b) a[b] += red[(w * NB + b) * 64 + lane];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int t = t0 + 16 * b + lr;
        if (t >= M) continue;
        const size_t o = (size_t)t * ldz + 16 * I + 4 * lg;
        if (ODT == TCQ_F32) {
            *gptr((float4_t*)((float*)S.out + o)) = float4_t{a[b][0] * rsv[0], a[b][1] * rsv[1], a[b][2] * rsv[2], a[b][3] * rsv[3]};
        } else {
            const u32 lo = bf16x2(a[b][0], a[b][1]), hi = bf16x2(a[b][2], a[b][3]);
            *gptr((u64*)((u16*)S.out + o)) = (u64)lo | ((u64)hi << 32);
        }
    }
}

// =========================================================================================================== C ABI
template <int MODE, int NB, int HL, bool RB>
static void launch_f_nb(int nseg, int rows, int odt, hipStream_t st, const FSegPack& P, const u16* h, int M, int K, int ldh, int ldz) {
    const int nch = (K + 255) / 256, maxw = FWaves<NB, HL>::max, nw = nch < maxw ? nch : maxw;
    const dim3 grid(rows, nseg, (M + 16 * NB - 1) / (16 * NB)), block(64 * nw);
    if (odt == TCQ_F32) launch_k(k_gemmf_small<MODE, NB, TCQ_F32, HL, RB>, grid, block, 0, st, P, h, M, K, ldh, ldz);
    else launch_k(k_gemmf_small<MODE, NB, TCQ_BF16, HL, RB>, grid, block, 0, st, P, h, M, K, ldh, ldz);
}
template <int MODE, int HL, bool RB = false>
static void launch_f(int nseg, int rows, int odt, hipStream_t st, const FSegPack& P, const u16* h, int M, int K, int ldh, int ldz) {
    if (M <= 16) launch_f_nb<MODE, 1, HL, RB>(nseg, rows, odt, st, P, h, M, K, ldh, ldz);
    else if (M <= 32) launch_f_nb<MODE, 2, HL, RB>(nseg, rows, odt, st, P, h, M, K, ldh, ldz);
    else launch_f_nb<MODE, 4, HL, RB>(nseg, rows, odt, st, P, h, M, K, ldh, ldz);
}

template <int MODE>
static int gemmf(const tcq_gemm_seg* segs, int nseg, const void* h, int M, int K, int odt, int ldo, tcq_stream_t stream) {
    if (!segs || !h || nseg <= 0 || M <= 0 || K <= 0 || ldo <= 0) return TCQ_ERR_ARG;
    if (odt != TCQ_F32 && odt != TCQ_BF16) return TCQ_ERR_DTYPE;
    if (nseg > TCQ_MAX_SEGS) return TCQ_ERR_UNSUPPORTED;
    if (K % 16) return TCQ_ERR_SHAPE;
    if ((size_t)M * K * 2 >= ((size_t)1 << 31) || (size_t)M * ldo >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
    if (ldo % 4 || (uintptr_t)h % 16) return TCQ_ERR_ALIGN;
    FSegPack P = {};
    int max_m = 0;
    for (int i = 0; i < nseg; ++i) {
        const tcq_gemm_seg& g = segs[i];
        if (!g.w || !g.out || (MODE == 0 && !g.t8) || (odt == TCQ_F32 && !g.rs) || g.m <= 0) return TCQ_ERR_ARG;
        if (g.m % 16) return TCQ_ERR_SHAPE;
        if (g.rows_per_table < 0 || (g.rows_per_table > 0 && (g.rows_per_table % 16 || g.m % g.rows_per_table))) return TCQ_ERR_SHAPE;
        if ((size_t)g.m * K >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
        if ((uintptr_t)g.out % (odt == TCQ_F32 ? 16 : 8) || (g.rs && (uintptr_t)g.rs % 16)) return TCQ_ERR_ALIGN;
        P.s[i] = g;
        if (g.m > max_m) max_m = g.m;
    }
    launch_f<MODE, HL_ROWS>(nseg, max_m / 16, odt, (hipStream_t)stream, P, (const u16*)h, M, K, 0, ldo);
    return launch_status();
}

extern "C" int tcq_gemmf_tcq(const tcq_gemm_seg* segs, int nseg, const void* h, int M, int K, int out_dtype, int ldo,
                             tcq_stream_t stream) {
    return gemmf<0>(segs, nseg, h, M, K, out_dtype, ldo, stream);
}

extern "C" int tcq_gemmf_w8(const tcq_gemm_seg* segs, int nseg, const void* h, int M, int K, int out_dtype, int ldo,
                            tcq_stream_t stream) {
    return gemmf<1>(segs, nseg, h, M, K, out_dtype, ldo, stream);
}

// ------------------------------------------------------------------------------------------ reference-shaped helpers
// kernels.gemmf_w8 / gemmf_tcq (deploy/tcq_kernels/kernels.py:689-696): activations hT (K, ldh) BF16 with token = column (as
// pre_h writes them), z (M, N) FP32 = acc * rs. The fused decode reads the stored words and picks table i of t8 (up to three
// concatenated (512, 2) tables) for tile rows I with (I >= nb0) + (I >= nb1) == i (k_gemmf_tcq, kernels.py:465-470).
static int f_cols_check(const void* w, const void* hT, int ldh, const float* rs, const float* z, int M, int N, int K) {
    if (!w || !hT || !rs || !z || M <= 0 || N <= 0 || K <= 0 || ldh < M) return TCQ_ERR_ARG;
    if (N % 16 || K % 16) return TCQ_ERR_SHAPE;
    if ((size_t)N * K >= ((size_t)1 << 31) || (size_t)K * ldh * 2 >= ((size_t)1 << 31) || (size_t)M * N >= ((size_t)1 << 31))
        return TCQ_ERR_SHAPE;
    if ((uintptr_t)z % 16 || (uintptr_t)rs % 16 || (uintptr_t)hT % 2) return TCQ_ERR_ALIGN;
    return TCQ_OK;
}

extern "C" int tcq_gemmf_w8_hT(const int8_t* W, const void* hT, int ldh, const float* rs, float* z, int M, int N, int K,
                               tcq_stream_t stream) {
    const int e = f_cols_check(W, hT, ldh, rs, z, M, N, K);
    if (e) return e;
    FSegPack P = {};
    P.s[0] = tcq_gemm_seg{W, nullptr, rs, z, N, 0};
    launch_f<1, HL_COLS>(1, N / 16, TCQ_F32, (hipStream_t)stream, P, (const u16*)hT, M, K, ldh, N);
    return launch_status();
}

extern "C" int tcq_gemmf_tcq_hT(const void* bits, const int8_t* t8, const void* hT, int ldh, const float* rs, float* z, int M, int N,
                                int K, int nb0, int nb1, tcq_stream_t stream) {
    const int e = f_cols_check(bits, hT, ldh, rs, z, M, N, K);
    if (e) return e;
    if (!t8 || nb0 < 0 || nb1 < nb0) return TCQ_ERR_ARG;
    const int tiles = N / 16, tiles_n = K / 16;
    const int bnd[4] = {0, nb0 < tiles ? nb0 : tiles, nb1 < tiles ? nb1 : tiles, tiles};
    FSegPack P = {};
    int nseg = 0, max_m = 0;
    for (int i = 0; i < 3; ++i) {
        const int lo = bnd[i], hi = bnd[i + 1];
        if (hi <= lo) continue;
        P.s[nseg++] = tcq_gemm_seg{(const u16*)bits + (size_t)lo * tiles_n * 32, t8 + 1024 * i, rs + 16 * lo, z + 16 * lo, 16 * (hi - lo), 0};
        if (16 * (hi - lo) > max_m) max_m = 16 * (hi - lo);
    }
    launch_f<0, HL_COLS, true>(nseg, max_m / 16, TCQ_F32, (hipStream_t)stream, P, (const u16*)hT, M, K, ldh, N);
    return launch_status();
}
