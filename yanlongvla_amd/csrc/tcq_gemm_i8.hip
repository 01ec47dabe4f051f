// W8A8 INT8 GEMM for many tokens on v_mfma_i32_16x16x64_i8: acc[m, n] = sum_k a[m, k] w[n, k] (exact int32), written as
// int32, as FP32 (float(acc) * sa[m]) * sw[n], or as BF16 of that. a (M, K) and w (N, K) are both row-major with K
// contiguous, so every MFMA operand is 16 consecutive bytes of one row.
//
// Workgroup tile TN weights x TM tokens, 4 waves in a 2 x 2 grid, each wave (TN / 2) x (TM / 2) = (TN / 32) x (TM / 32)
// MFMA blocks. MFMA A = weight rows (lane (g, r): row r, k-block g), B = token rows, D: lane (g, t) holds weights
// 4 g .. 4 g + 3 of token t -> 4 consecutive output columns, one 16-byte store.
// K steps of 64: the next step's A / W tiles are loaded into registers (buffer loads; rows past M / N and columns past K
// read zeros) while the current step multiplies from LDS; tiles in LDS are 64-byte rows with the 16-byte granules swizzled
// by (row >> 2) so that the 16 rows of a fragment read hit 16 different bank groups.
#include "tcq_device.h"
#include "tcq_launch.h"

namespace {

typedef int int4v __attribute__((ext_vector_type(4)));
constexpr int GT = 256;   // threads per workgroup

__device__ __forceinline__ int swz(int row, int g) { return row * 64 + 16 * (g ^ ((row >> 2) & 3)); }

}  // namespace

template <int TN, int TM, int ODT>
__global__ __launch_bounds__(GT) void k_gemm_i8(const i8* a, const i8* w, const float* sa, const float* sw, void* out, int ldo,
                                                int M, int N, int K) {
    constexpr int GR = (TN + TM) * 4 / GT;                 // 16-byte granules per thread per K step
    constexpr int BN = TN / 32, BM = TM / 32;              // MFMA blocks per wave
    __shared__ __attribute__((aligned(16))) char sw_t[2][TN * 64];
    __shared__ __attribute__((aligned(16))) char sa_t[2][TM * 64];
    const int n0 = blockIdx.x * TN, m0 = blockIdx.y * TM;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int wn = wave & 1, wm = wave >> 1, lr = lane & 15, lg = lane >> 4;
    const rsrc_t RA = make_rsrc(a, (u32)M * (u32)K), RW = make_rsrc(w, (u32)N * (u32)K);
    const int nk = (K + 63) >> 6;

    // staging: granule gi of the step = (row, g): rows 0..TN-1 of w then 0..TM-1 of a
    uint4_t st[GR];
    auto gload = [&](int kt) {
#pragma unroll
        for (int p = 0; p < GR; ++p) {
            const int gi = threadIdx.x + p * GT, row = gi >> 2, g = gi & 3, k = 64 * kt + 16 * g;
            if (row < TN) {
                const u32 off = (n0 + row < N && k < K) ? (u32)(n0 + row) * (u32)K + (u32)k : RSRC_OOB;
                st[p] = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(RW, off, 0, 2));
            } else {
                const int r = row - TN;
                const u32 off = (m0 + r < M && k < K) ? (u32)(m0 + r) * (u32)K + (u32)k : RSRC_OOB;
                st[p] = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(RA, off, 0, 0));
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int p = 0; p < GR; ++p) {
            const int gi = threadIdx.x + p * GT, row = gi >> 2, g = gi & 3;
            if (row < TN) *(uint4_t*)(sw_t[buf] + swz(row, g)) = st[p];
            else *(uint4_t*)(sa_t[buf] + swz(row - TN, g)) = st[p];
        }
    };

    int4v acc[BN][BM];
#pragma unroll
    for (int i = 0; i < BN; ++i)
#pragma unroll
        for (int j = 0; j < BM; ++j) acc[i][j] = int4v{0, 0, 0, 0};

    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
        int4v A[BN], B[BM];
#pragma unroll
        for (int i = 0; i < BN; ++i) A[i] = *(const int4v*)(sw_t[cur] + swz(wn * (TN / 2) + 16 * i + lr, lg));
#pragma unroll
        for (int j = 0; j < BM; ++j) B[j] = *(const int4v*)(sa_t[cur] + swz(wm * (TM / 2) + 16 * j + lr, lg));
#pragma unroll
        for (int i = 0; i < BN; ++i)
#pragma unroll
            for (int j = 0; j < BM; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[i], B[j], acc[i][j], 0, 0, 0);
        if (kt + 1 < nk) lstore(cur ^ 1);
        __syncthreads();
    }

    // epilogue: lane (g, t) of block (i, j) holds weights n = n0 + wn TN/2 + 16 i + 4 g .. + 3 of token m = m0 + wm TM/2 + 16 j + t
#pragma unroll
    for (int i = 0; i < BN; ++i) {
        const int n = n0 + wn * (TN / 2) + 16 * i + 4 * lg;
        if (n >= N) continue;
        float4_t swv = {0.f, 0.f, 0.f, 0.f};
        if (ODT != TCQ_I32) swv = gptr((const float4_t*)(sw + n))[0];
#pragma unroll
        for (int j = 0; j < BM; ++j) {
            const int m = m0 + wm * (TM / 2) + 16 * j + lr;
            if (m >= M) continue;
            const size_t o = (size_t)m * ldo + n;
            if (ODT == TCQ_I32) {
                *gptr((int4v*)((int*)out + o)) = acc[i][j];
            } else {
                const float s = gptr(sa)[m];
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = ((float)acc[i][j][e] * s) * swv[e];
                if (ODT == TCQ_F32) *gptr((float4_t*)((float*)out + o)) = float4_t{v[0], v[1], v[2], v[3]};
                else {
                    const u32 lo = (u32)f32_to_bf16(v[0]) | ((u32)f32_to_bf16(v[1]) << 16);
                    const u32 hi = (u32)f32_to_bf16(v[2]) | ((u32)f32_to_bf16(v[3]) << 16);
                    *gptr((u64*)((u16*)out + o)) = (u64)lo | ((u64)hi << 32);
                }
            }
        }
    }
}

// =========================================================================================================== C ABI
extern "C" int tcq_gemm_i8(const int8_t* a, const int8_t* w, const float* sa, const float* sw, void* out, int out_dtype, int ldo,
                           int M, int N, int K, tcq_stream_t stream) {
    if (!a || !w || !out || M <= 0 || N <= 0 || K <= 0 || ldo < N) return TCQ_ERR_ARG;
    if (out_dtype != TCQ_I32 && (!sa || !sw)) return TCQ_ERR_ARG;
    if (K % 16 || N % 4) return TCQ_ERR_SHAPE;
    if ((size_t)M * K >= ((size_t)1 << 31) || (size_t)N * K >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
    if ((uintptr_t)a % 16 || (uintptr_t)w % 16 || (uintptr_t)out % 16 || (sw && (uintptr_t)sw % 16) || ldo % 4)
        return TCQ_ERR_ALIGN;
    hipStream_t st = (hipStream_t)stream;
    constexpr int TN = 128, TM = 128;
    const dim3 grid((N + TN - 1) / TN, (M + TM - 1) / TM), block(GT);
    switch (out_dtype) {
        case TCQ_I32: launch_k(k_gemm_i8<TN, TM, TCQ_I32>, grid, block, 0, st, (const i8*)a, (const i8*)w, sa, sw, out, ldo, M, N, K); break;
        case TCQ_F32: launch_k(k_gemm_i8<TN, TM, TCQ_F32>, grid, block, 0, st, (const i8*)a, (const i8*)w, sa, sw, out, ldo, M, N, K); break;
        case TCQ_BF16: launch_k(k_gemm_i8<TN, TM, TCQ_BF16>, grid, block, 0, st, (const i8*)a, (const i8*)w, sa, sw, out, ldo, M, N, K); break;
        default: return TCQ_ERR_DTYPE;
    }
    return launch_status();
}
