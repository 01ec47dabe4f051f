// GEMM for many tokens, acc[m, n] = sum_k a[m, k] w[n, k], a (M, K) and w (N, K) both row-major with K contiguous, so every
// MFMA operand is 16 consecutive bytes of one row:
//   INT8 (W8A8) on v_mfma_i32_32x32x32_i8 (measured on MI355X: 4.05 POPS for back-to-back independent 32 x 32 x 32 products
//   against 2.7 for 16 x 16 x 64): exact int32 acc, written as int32, as FP32 (float(acc) * sa[m]) * sw[n], or as BF16 of
//   that;
//   BF16 (the W2 float path: BF16 rotated activations times the INT8 table values as BF16) on v_mfma_f32_32x32x16_bf16 with
//   FP32 accumulation, written as FP32 (acc * sa[m]) * sw[n] (either scale may be absent) or as BF16 of that.
// Both take 64-byte K steps: 64 int8 = two 32-element MFMA halves, or 32 bf16 = two 16-element MFMA steps, with the same
// 16-byte fragment per lane.
//
// Workgroup tile TN weights x TM tokens, WN x WM waves, each (TN / WN) x (TM / WM) in 32 x 32 MFMA blocks. MFMA A = 32
// token rows (lane (h, r): row r, 16 columns of half h of the 32), B = 32 weight rows, D: register 4 q + e of lane (h, c)
// holds token 8 q + 4 h + e of weight c, so the 32 lanes of a half store 32 consecutive output columns.
// K steps of 64 bytes go HBM -> LDS by buffer_load_dwordx4 ... lds (no registers), NS steps in flight: the loads of step
// kt + NS - 1 are issued right after the barrier that opens step kt. A step holds 1 KiB blocks of 16 rows x 64 bytes; lane
// p of a load writes position p of its block, which holds row p / 4 and 16-byte granule (p % 4) ^ ((row / 4) % 4), so the
// 16 rows of a fragment read hit 16 different bank groups. Rows past M / N and columns past K read zeros.
#include "tcq_device.h"
#include "tcq_launch.h"

namespace {

typedef int int4v __attribute__((ext_vector_type(4)));
typedef int int16v __attribute__((ext_vector_type(16)));

__device__ __forceinline__ int swz(int row, int g) { return row * 64 + 16 * (g ^ ((row >> 2) & 3)); }

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding: vmcnt bits 3:0 and 15:14)
template <int n>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier without the memory fence of __syncthreads (which waits for every outstanding load, including the LDS
// loads of later steps): the LDS writes a barrier must publish are the loads waited for just before it (wait_vm), and the
// empty asm statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void barrier_nofence() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

}  // namespace

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

template <int ESZ> struct MfmaOf;
template <> struct MfmaOf<1> {                 // INT8
    typedef int16v acc_t;
    static __device__ __forceinline__ acc_t mma(int4v a, int4v b, acc_t c) { return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0); }
};
template <> struct MfmaOf<2> {                 // BF16
    typedef float16v acc_t;
    static __device__ __forceinline__ acc_t mma(int4v a, int4v b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
};

// ESZ: element size (1 INT8, 2 BF16); K in elements. WAUX: cache policy of the weight loads, non-temporal (2) when a single
// tile row of tokens reads every weight once, temporal (0) when several token tiles reread them (measured at M = 800,
// N = 16384, K = 2048: 40.6 against 46.3 us per launch; the four token tiles of a weight tile run on one XCD and share its L2).
template <int ESZ, int TN, int TM, int WN, int WM, int NS, int ODT, int WAUX = 2>
__global__ __launch_bounds__(64 * WN * WM) void k_gemm_i8(const void* a_, const void* w_, const float* sa, const float* sw, void* out,
                                                          int ldo, int M, int N, int K_) {
    typedef typename MfmaOf<ESZ>::acc_t acc_t;
    const char* a = (const char*)a_;
    const char* w = (const char*)w_;
    const int K = K_ * ESZ;                                              // row length in bytes
    constexpr int NWAVE = WN * WM;
    constexpr int WBLK = TN / 16, ABLK = TM / 16, BLK = WBLK + ABLK;    // 1 KiB blocks (16 rows x 64 bytes) per step
    constexpr int PW = BLK / NWAVE;                                      // direct loads per wave per step
    constexpr int BN = TN / WN / 32, BM = TM / WM / 32;                  // 32 x 32 MFMA blocks per wave
    static_assert(BLK % NWAVE == 0 && TN % (32 * WN) == 0 && TM % (32 * WM) == 0, "tile shape");
    __shared__ __attribute__((aligned(1024))) char lds[NS][BLK * 1024];
    const int n0 = blockIdx.x * TN, m0 = blockIdx.y * TM;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int wn = wave % WN, wm = wave / WN;
    const int l32 = lane & 31, lh = lane >> 5;                           // MFMA operand lane: row l32, k-half lh
    const rsrc_t RA = make_rsrc(a, (u32)M * (u32)K), RW = make_rsrc(w, (u32)N * (u32)K);
    const int nk = (K + 63) >> 6;
    const int prow = lane >> 2, pg = (lane & 3) ^ ((prow >> 2) & 3);  // what this lane loads in a block

    auto issue = [&](int kt) {
        char* st = lds[kt % NS];
        const int k = 64 * kt + 16 * pg;
#pragma unroll
        for (int u = 0; u < PW; ++u) {
            const int blk = wave * PW + u;
            char* dst = st + blk * 1024;
            if (blk < WBLK) {
                const int row = n0 + 16 * blk + prow;
                const u32 off = (row < N && k < K) ? (u32)row * (u32)K + (u32)k : RSRC_OOB;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(RW, (__attribute__((address_space(3))) void*)dst, 16, off, 0, 0, WAUX);
            } else {
                const int row = m0 + 16 * (blk - WBLK) + prow;
                const u32 off = (row < M && k < K) ? (u32)row * (u32)K + (u32)k : RSRC_OOB;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(RA, (__attribute__((address_space(3))) void*)dst, 16, off, 0, 0, 0);
            }
        }
    };
    // fragment of 32 rows starting at 16-row block b0, k half kk (columns 32 kk .. 32 kk + 31 of the step)
    auto frag = [&](const char* st, int b0, int kk) {
        return *(const int4v*)(st + (b0 + (l32 >> 4)) * 1024 + swz(l32 & 15, 2 * kk + lh));
    };

    acc_t acc[BN][BM];
#pragma unroll
    for (int i = 0; i < BN; ++i)
#pragma unroll
        for (int j = 0; j < BM; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

#pragma unroll
    for (int t = 0; t < NS - 1; ++t)
        if (t < nk) issue(t);
    for (int kt = 0; kt < nk; ++kt) {
        if (kt + NS - 2 < nk) wait_vm<(NS - 2) * PW>();                 // this wave's loads of step kt have landed
        else wait_vm<0>();
        barrier_nofence();                                               // ... and every other wave's
        if (kt + NS - 1 < nk) issue(kt + NS - 1);                        // into the buffer of step kt - 1 (all done with it)
        const char* st = lds[kt % NS];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            int4v A[BM], B[BN];
#pragma unroll
            for (int j = 0; j < BM; ++j) A[j] = frag(st, WBLK + (wm * BM + j) * 2, kk);
#pragma unroll
            for (int i = 0; i < BN; ++i) B[i] = frag(st, (wn * BN + i) * 2, kk);
#pragma unroll
            for (int j = 0; j < BM; ++j)
                // blocks of padding rows only: no MFMA work (with one wave row, where a tile always holds rows, the test is
                // left out: the branch changed the code of the narrow tiles and slowed them)
                if (WM == 1 || m0 + (wm * BM + j) * 32 < M)
#pragma unroll
                    for (int i = 0; i < BN; ++i) acc[i][j] = MfmaOf<ESZ>::mma(A[j], B[i], acc[i][j]);
        }
    }

    // epilogue: block (i, j), register 4 q + e of lane (lh, l32) = token m0 + (wm BM + j) 32 + 8 q + 4 lh + e, weight
    // n0 + (wn BN + i) 32 + l32.
    if constexpr (ODT == TCQ_I32) {
        // the 32 lanes of a half store 32 consecutive int32 columns: whole 128-byte lines
#pragma unroll
        for (int j = 0; j < BM; ++j) {
            const int mb = m0 + (wm * BM + j) * 32 + 4 * lh;
#pragma unroll
            for (int i = 0; i < BN; ++i) {
                const int n = n0 + (wn * BN + i) * 32 + l32;
                if (n >= N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = mb + 8 * (r >> 2) + (r & 3);
                    if (m < M) gptr((int*)out)[(size_t)m * ldo + n] = (int)acc[i][j][r];
                }
            }
        }
    } else {
        // FP32 / BF16: each wave stages one 32-token block row of its tile at a time in its own slice of the (now idle) LDS
        // ring, row-major, and stores it back as 16-byte pieces of whole row segments (2-byte scattered stores of BF16
        // leave half lines and run at a fraction of the bandwidth).
        constexpr int OSZ = ODT == TCQ_BF16 ? 2 : 4;
        constexpr int WTN = TN / WN, RB = WTN * OSZ, GPR = RB / 16, EPG = 16 / OSZ;
        constexpr int SLICE = NS * BLK * 1024 / NWAVE;
        static_assert(32 * RB <= SLICE, "epilogue staging slice");
        __syncthreads();                                                 // every wave is done with the ring
        char* slice = &lds[0][0] + wave * SLICE;
        const int nw0 = n0 + wn * WTN;
        const bool vec = ((size_t)ldo * OSZ) % 16 == 0 && ((uintptr_t)out % 16) == 0;
        float swv[BN];
#pragma unroll
        for (int i = 0; i < BN; ++i) {
            const int n = nw0 + i * 32 + l32;
            swv[i] = (sw && n < N) ? gptr(sw)[n] : 1.f;
        }
#pragma unroll
        for (int j = 0; j < BM; ++j) {
            const int mb = m0 + (wm * BM + j) * 32;
            float sam[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = mb + 8 * (r >> 2) + 4 * lh + (r & 3);
                sam[r] = (sa && m < M) ? gptr(sa)[m] : 1.f;
            }
#pragma unroll
            for (int i = 0; i < BN; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int tr = 8 * (r >> 2) + 4 * lh + (r & 3);
                    const float v = ESZ == 1 ? ((float)acc[i][j][r] * sam[r]) * swv[i]
                                             : (sa ? (float)acc[i][j][r] * sam[r] : (float)acc[i][j][r]) * (sw ? swv[i] : 1.f);
                    char* dst = slice + tr * RB + (i * 32 + l32) * OSZ;
                    if (ODT == TCQ_F32) *(float*)dst = v;
                    else *(u16*)dst = f32_to_bf16(v);
                }
            constexpr int NG = (32 * GPR + 63) / 64;                     // 16-byte pieces per lane (a fixed count: unrolled)
#pragma unroll
            for (int it = 0; it < NG; ++it) {
                const int g = lane + 64 * it;
                const int tr = g / GPR, cg = g - tr * GPR;
                const int m = mb + tr, n = nw0 + cg * EPG;
                if (g >= 32 * GPR || m >= M || n >= N) continue;
                const uint4_t v = *(const uint4_t*)(slice + tr * RB + cg * 16);
                char* o = (char*)out + ((size_t)m * ldo + n) * OSZ;
                if (vec && n + EPG <= N) {
                    *gptr((uint4_t*)o) = v;
                } else {                                                 // row end or unaligned rows: element stores
#pragma unroll
                    for (int e = 0; e < EPG; ++e) {
                        if (n + e >= N) break;
                        const u32 word = v[e * OSZ / 4];
                        if (OSZ == 2) gptr((u16*)o)[e] = (u16)(word >> (16 * (e & 1)));
                        else gptr((u32*)o)[e] = word;
                    }
                }
            }
        }
    }
}

// =========================================================================================================== C ABI
template <int ESZ, int TN, int TM, int WN, int WM, int NS>
static void launch_gemm(int odt, hipStream_t st, const void* a, const void* w, const float* sa, const float* sw, void* out, int ldo,
                        int M, int N, int K) {
    const dim3 grid((N + TN - 1) / TN, (M + TM - 1) / TM), block(64 * WN * WM);
    if (grid.y > 1) {                                   // token tiles share each weight tile: keep the weights in L2
        if (odt == TCQ_I32) launch_k(k_gemm_i8<ESZ, TN, TM, WN, WM, NS, TCQ_I32, 0>, grid, block, 0, st, a, w, sa, sw, out, ldo, M, N, K);
        else if (odt == TCQ_F32) launch_k(k_gemm_i8<ESZ, TN, TM, WN, WM, NS, TCQ_F32, 0>, grid, block, 0, st, a, w, sa, sw, out, ldo, M, N, K);
        else launch_k(k_gemm_i8<ESZ, TN, TM, WN, WM, NS, TCQ_BF16, 0>, grid, block, 0, st, a, w, sa, sw, out, ldo, M, N, K);
        return;
    }
    if (odt == TCQ_I32) launch_k(k_gemm_i8<ESZ, TN, TM, WN, WM, NS, TCQ_I32>, grid, block, 0, st, a, w, sa, sw, out, ldo, M, N, K);
    else if (odt == TCQ_F32) launch_k(k_gemm_i8<ESZ, TN, TM, WN, WM, NS, TCQ_F32>, grid, block, 0, st, a, w, sa, sw, out, ldo, M, N, K);
    else launch_k(k_gemm_i8<ESZ, TN, TM, WN, WM, NS, TCQ_BF16>, grid, block, 0, st, a, w, sa, sw, out, ldo, M, N, K);
}

template <int ESZ>
static void launch_by_m(int odt, hipStream_t st, const void* a, const void* w, const float* sa, const float* sw, void* out, int ldo,
                        int M, int N, int K) {
    // The largest tile (weights x tokens) that still gives one workgroup per CU (256), else the smallest: a narrow product
    // on 256 x 256 tiles leaves most CUs idle. Measured on MI355X at M = 800 (FP32 out, bit-identical across tiles):
    // N = 2048, K = 16384: 206.5 us on 256 x 256 (32 workgroups), 84.3 on 128 x 64 (208); N = 2048, K = 2048: 32.3 -> 15.4;
    // N = 2560: 37.9 -> 16.8; N = 32768 (512 workgroups of 256 x 256): 118.5 against 143-274 on the smaller tiles.
    auto wgs = [&](int tn, int tm) { return (long)((N + tn - 1) / tn) * ((M + tm - 1) / tm); };
    if (M > 128 && wgs(256, 256) >= 256) launch_gemm<ESZ, 256, 256, 2, 4, 4>(odt, st, a, w, sa, sw, out, ldo, M, N, K);
    else if (M > 64 && wgs(256, 128) >= 256) launch_gemm<ESZ, 256, 128, 4, 2, 4>(odt, st, a, w, sa, sw, out, ldo, M, N, K);
    else if (wgs(256, 64) >= 256) launch_gemm<ESZ, 256, 64, 4, 1, 4>(odt, st, a, w, sa, sw, out, ldo, M, N, K);
    else launch_gemm<ESZ, 128, 64, 4, 1, 4>(odt, st, a, w, sa, sw, out, ldo, M, N, K);
}

extern "C" int tcq_gemm_i8(const int8_t* a, const int8_t* w, const float* sa, const float* sw, void* out, int out_dtype, int ldo,
                           int M, int N, int K, tcq_stream_t stream) {
    if (!a || !w || !out || M <= 0 || N <= 0 || K <= 0 || ldo < N) return TCQ_ERR_ARG;
    if (out_dtype != TCQ_I32 && (!sa || !sw)) return TCQ_ERR_ARG;
    if (K % 16 || N % 4) return TCQ_ERR_SHAPE;
    if ((size_t)M * K >= ((size_t)1 << 31) || (size_t)N * K >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
    if ((uintptr_t)a % 16 || (uintptr_t)w % 16 || (uintptr_t)out % 16 || (sw && (uintptr_t)sw % 16) || ldo % 4)
        return TCQ_ERR_ALIGN;
    if (M <= 16 || (M <= 64 && N <= 8192)) {            // few tokens: the small-M product (one K chunk per wave)
        const tcq_gemm_seg seg = {w, nullptr, sw, out, N};
        if (N % 16 == 0) return tcq_gemm_w8(&seg, 1, a, sa, M, K, out_dtype, ldo, stream);
    }
    if (out_dtype != TCQ_I32 && out_dtype != TCQ_F32 && out_dtype != TCQ_BF16) return TCQ_ERR_DTYPE;
    launch_by_m<1>(out_dtype, (hipStream_t)stream, a, w, sa, sw, out, ldo, M, N, K);
    return launch_status();
}

extern "C" int tcq_gemm_bf16(const void* a, const void* w, const float* sa, const float* sw, void* out, int out_dtype, int ldo, int M,
                             int N, int K, tcq_stream_t stream) {
    if (!a || !w || !out || M <= 0 || N <= 0 || K <= 0 || ldo < N) return TCQ_ERR_ARG;
    if (out_dtype != TCQ_F32 && out_dtype != TCQ_BF16) return TCQ_ERR_DTYPE;
    if (K % 16 || N % 4) return TCQ_ERR_SHAPE;
    if ((size_t)M * K * 2 >= ((size_t)1 << 31) || (size_t)N * K * 2 >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
    if ((uintptr_t)a % 16 || (uintptr_t)w % 16 || (uintptr_t)out % 16 || (sw && (uintptr_t)sw % 16) || ldo % 4) return TCQ_ERR_ALIGN;
    launch_by_m<2>(out_dtype, (hipStream_t)stream, a, w, sa, sw, out, ldo, M, N, K);
    return launch_status();
}
