// Small-M INT8 products (M <= 64 tokens) on v_mfma_i32_16x16x64_i8: the W2A8 fused trellis decode + product, and the same
// product on resident INT8 weights. z[t, i] = (float(acc[t, i]) * s[t]) * rs[i], acc exact in int32 (the reference's
// finish(), deploy/tcq_kernels/kernels.py:355-363).
//
// MFMA mapping per 256-column chunk c and j = 0..3: A = weights, lane (g, r) = row r of the tile row, k-block g = the 16
// columns of tile 16 c + 4 j + g (exactly one decoded tile row per lane); B = activations, lane (g, t) = token t of the
// token block, the same 16 columns; D: lane (g, t) holds rows 4 g .. 4 g + 3 of token t.
// A from the trellis words: the window layout of tcq_repack (one dwordx4 per lane per tile row and chunk), 8 lookups of
// INT8 pairs in a sign-folded LDS table (1024 entries x SM_C copies, one 4-byte slot each, lane l reads copy l mod SM_C),
// packed into the 16 A bytes. A from resident INT8 weights: one 16-byte load per lane per (tile row, j).
// Work split (few tokens = little work per layer, so the launch is latency-bound): a workgroup takes one tile row (16 output
// rows) of one segment and its waves split K, one 256-column chunk each (up to 16 waves; wave w takes chunks w, w + NW, ...
// beyond 16 chunks). Every wave issues the loads of its words / weights and of its activation fragments (16 bytes of each
// token per lane and j, straight into registers; zero for tokens >= M and columns >= K) before the table fill, so a
// workgroup costs one memory round trip. The partial int32 sums of the waves are added in LDS at the end (exact).
#include "tcq_device.h"
#include "tcq_launch.h"
#include "tcq_rows.h"
#include "tcq_attend.h"

namespace {

constexpr int SM_C = 4;                // table copies (a workgroup streams little: the fill must stay cheap)
constexpr int SM_MAXW = 16;            // waves per workgroup at most

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

// acc + the dot product of the 16 INT8 weights a with the 16 INT8 activations b (four v_dot4c_i32_i8; exact int32).
__device__ __forceinline__ int dot_product(int4v a, int4v b, int acc) {
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_sdot4(a[e], b[e], acc, false);
    return acc;
}

// One-token dot products -> the MFMA result layout: v is lane (g, r)'s sum over k-block g of row r (token 0); the four
// k-blocks are added (exact), and lane (g, 0) receives rows 4 g .. 4 g + 3 as the 16 x 16 x 64 MFMA leaves token 0
// (every other lane: zeros, as the MFMA's empty token columns).
__device__ __forceinline__ int4v dot_to_mfma_layout(int v, int lane) {
    v += __float_as_int(lane_xor(__int_as_float(v), 16, lane));
    v += __float_as_int(lane_xor(__int_as_float(v), 32, lane));
    int4v o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int x = __builtin_amdgcn_ds_bpermute((4 * (lane >> 4) + e) << 2, v);
        o[e] = (lane & 15) ? 0 : x;
    }
    return o;
}

}  // namespace

struct SegPack {
    tcq_gemm_seg s[TCQ_MAX_SEGS];
};

// The segments plus the arguments of a one-token prologue (tcq_gemm_tcq_pro / tcq_gemm_w8_pro).
struct SegPackPro {
    tcq_gemm_seg s[TCQ_MAX_SEGS];
    PanpArgs a;
    i8* q;                   // optional copies of the prologue's INT8 row and token scale (written by workgroup 0)
    float* scale;
    const float* part;       // attention partials (PRO_ATTN)
    int nc, keys, causal, heads;
};

// Prologue kinds (the PL template argument of the product kernels): PRO_LAYER, the decoder-layer prologue of a 2048-wide
// row (tcq_post_add_norm_pre's operations, 8 values per thread); PRO_PRE, the rotate + quantize of a 16384-wide BF16 row
// (tcq_pre's, 32 values per thread); PRO_ATTN, the attention chunk merge of 8 heads (k_attn_combine_w's, one wave per head)
// and the rotate + quantize of its 2048-wide row (8 values per thread). All on the register + transpose engine, as the
// standalone kernels run them.
enum { PRO_NONE = 0, PRO_LAYER = 1, PRO_PRE = 2, PRO_ATTN = 3 };
template <int PL> struct PackOf { typedef SegPackPro type; };
template <> struct PackOf<PRO_NONE> { typedef SegPack type; };
template <int PL> struct ProShape {
    static_assert(PL == PRO_LAYER || PL == PRO_PRE || PL == PRO_ATTN, "prologue kind");
    static constexpr int L = PL == PRO_PRE ? 14 : 11, LE = PL == PRO_PRE ? 5 : 3;
};

// LDS of a prologue: the Walsh engine's row, the chunk sums, the reduction slots, the INT8 row and its scale (the
// product's activations), and the attention merge's chunk weights.
template <int PL>
struct ProLds {
    static constexpr int N = 1 << ProShape<PL>::L;
    static constexpr int W = N + (N >> 5) + 1;                           // lds_words(N)
    float xs[W + N / 16];
    float red[16];
    __attribute__((aligned(16))) u32 qs[N / 4];
    float sc;
    float wts[PL == PRO_ATTN ? AH : 1][MAXC];
    WavesLds wl[PL == PRO_PRE ? 0 : 1];                                  // the eight-wave engine's exchange (NWP = 8)
};

// Runs the prologue and leaves the INT8 row and the scale in L; workgroup (0, 0, 0) stores the side outputs (xout, the
// optional q / scale copies). Every thread of the workgroup calls it; mid() issues the product's weight loads once the
// prologue's entry loads have been consumed, so their HBM latency runs under the prologue.
// NWP = 8 (workgroups of exactly eight waves; the layer and attention prologues): the 2048-wide row on all eight waves,
// four values per thread, on panp_waves / waves_rotate_quantize (no LDS transposes); the same row and scale.
template <int PL, int NWP = 0, class F>
__device__ __forceinline__ void run_prologue(const SegPackPro& P, ProLds<PL>& L, F&& mid) {
    constexpr int NL = ProShape<PL>::L, LE = ProShape<PL>::LE;
    const bool store = blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0;
    if constexpr (NWP == 8) {
        static_assert(PL == PRO_LAYER || PL == PRO_ATTN, "eight-wave prologue: 2048-wide rows");
        const auto bar = [] { __syncthreads(); };
        float v[4];
        if constexpr (PL == PRO_LAYER) {
            panp_waves<TCQ_I32, 8>(P.a, 0, store, v, L.wl[0], mid, bar);
        } else {
            combine_w_row(P.part, P.nc, P.keys, P.causal, P.heads, 0, nullptr, P.a.su, L.xs, L.wts, mid, v);   // heads = 8
        }
        waves_rotate_quantize<8>(v, L.wl[0], L.qs, &L.sc, store ? P.q : nullptr, store ? P.scale : nullptr, bar);
        return;
    }
    float v[1 << LE];
    if constexpr (PL == PRO_LAYER) {
        panp_tw<TCQ_I32, NL, LE, false>(P.a, 0, store, v, L.xs, L.xs + ProLds<PL>::W, L.red, mid);
    } else if constexpr (PL == PRO_PRE) {
        pre_row_tw<NL, LE>(P.a.x, P.a.su, v, mid);
    } else {
        combine_w_row(P.part, P.nc, P.keys, P.causal, P.heads, 0, nullptr, P.a.su, L.xs, L.wts, mid);
        tw_get<NL, LE, 0>(v, L.xs);
    }
    tw_rotate_quantize<NL, LE>(v, L.xs, L.red, store ? P.q : nullptr, nullptr, 0, store ? P.scale : nullptr, 0, L.qs, &L.sc);
}

// Activation layouts of the small-M products: q (M, K) row-major, the token-block layout, or the reference's q4 (K/4, ldq)
// int32 words (4 consecutive inputs of one token per word, token = column; deploy/tcq_kernels/kernels.py:170-184).
enum { QL_ROWS = 0, QL_BLOCKS = 1, QL_WORDS = 2 };

// grid (tile-row groups of the largest segment, segments), NW = blockDim.x / 64 waves; a workgroup takes TR consecutive tile
// rows (the activation fragments of its chunks, the bulk of the loads, then serve TR rows). MODE 0: decode from tcq_repack
// words (RB: from the reference word layout, 64 bytes per tile, tiles row-major); MODE 1: resident INT8 weights. ODT: output
// dtype (F32 scaled, BF16 scaled, I32 accumulators). QL: activation layout (ldq only for QL_WORDS).
// KS > 1 (I32 only): K parts, blockIdx.z = part p takes chunks [p * ceil(nch / KS), ...) and writes at out + p * M * ldz.
// DOT (M == 1): the product on v_dot4c_i32_i8 (dot_product) instead of the MFMA; the epilogues are shared.
// PL > 0 (M == 1, K = 2^PL): the activations come from the prologue run by every workgroup (run_prologue, ProShape)
// instead of q / s.
// OVS (the layer or attention prologue, one tile row, one chunk per product wave): the prologue runs on waves 0 .. 7
// while waves 8 .. NW - 1 fill the table and decode the weight fragments of their chunks (chunk c0 + wave - 8) into
// registers, meeting the prologue's barriers; after the row is in LDS they multiply, and their partial sums add in chunk
// order as without OVS (the same sums and outputs).
template <int MODE, int NB, int ODT, int TR, int QL, bool RB = false, int KS = 1, bool DOT = false, int PL = 0, bool OVS = false>
__global__ __launch_bounds__(TR == 1 ? 1024 : 512) void k_gemm_small(const typename PackOf<PL>::type P, const i8* q, const float* s,
                                                                    int M, int K, int ldz, int ldq) {
    static_assert(!OVS || ((PL == PRO_LAYER || PL == PRO_ATTN) && MODE == 0 && TR == 1 && !RB), "overlapped prologue");
    static_assert(KS == 1 || ODT == TCQ_I32, "K parts are int32 sums");
    static_assert(!DOT || (NB == 1 && QL != QL_WORDS), "dot products: one token, q rows or token blocks");
    static_assert(PL == 0 || (NB == 1 && QL == QL_ROWS && !DOT), "prologue: one token");
    __shared__ __attribute__((aligned(16))) u32 tab[MODE == 0 ? 1024 * SM_C : 4];
    __shared__ __attribute__((aligned(16))) int4v red[(TR == 1 ? SM_MAXW - 1 : 7) * TR * NB * 64];
    __shared__ ProLds<PL ? PL : PRO_LAYER> pro;
    const tcq_gemm_seg S = P.s[blockIdx.y];
    const int tiles_m = S.m >> 4, nch_all = (K + 255) >> 8;
    const int c0 = KS > 1 ? (int)blockIdx.z * ((nch_all + KS - 1) / KS) : 0;
    const int nch = KS > 1 ? min(nch_all, c0 + (nch_all + KS - 1) / KS) : nch_all;   // chunks c0 .. nch - 1
    const int I0 = blockIdx.x * TR;
    if (I0 >= tiles_m) return;                                            // uniform
    const int nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    // OVS: the product's waves are 8 .. nw - 1 (pw = wave - 8 of npw); otherwise every wave
    const int pw = OVS ? wave - 8 : wave, npw = OVS ? nw - 8 : nw;
    const int lr = lane & 15, lg = lane >> 4;
    const u32 cp4 = (u32)(lane & (SM_C - 1)) << 2;
    constexpr int ESH = SM_C == 16 ? 6 : SM_C == 8 ? 5 : SM_C == 4 ? 4 : 2;
    const int tiles_n = K >> 4;
    rsrc_t Wr;
    if (MODE == 0) Wr = make_rsrc(S.w, RB ? (u32)(tiles_m * tiles_n) << 6 : (u32)(tiles_m * nch_all) << 10);
    else Wr = make_rsrc(S.w, (u32)S.m * (u32)K);
    const rsrc_t Q = make_rsrc(q, QL == QL_BLOCKS ? (u32)((M + 15) >> 4) * 16u * (u32)K
                                  : QL == QL_WORDS ? (u32)(K >> 2) * (u32)ldq * 4u : (u32)M * (u32)K);

    uint4_t wa[TR][MODE == 0 ? 1 : 4];
    int4v B[4][NB];
    auto loadB = [&](int c) {                                             // activations of chunk c from the prologue's row
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = 256 * c + 64 * j + 16 * lg;
            B[j][0] = (lr < M && k < K) ? *(const int4v*)((const char*)pro.qs + k) : int4v{0, 0, 0, 0};
        }
    };
    auto load = [&](int c) {                                              // words / weights and activations of chunk c
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            const int I = min(I0 + r, tiles_m - 1);                       // a row past the end reloads the last (never stored)
            if (MODE == 0 && RB) {                                        // dword lr of tile 16 c + 4 j + lg, halves swapped
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int J = 16 * c + 4 * j + lg;
                    const u32 off = J < tiles_n ? (((u32)(I * tiles_n + J) << 6) | ((u32)lr << 2)) : RSRC_OOB;
                    const u32 d = __builtin_amdgcn_raw_buffer_load_b32(Wr, off, 0, 2);
                    wa[r][0][j] = __builtin_amdgcn_alignbit(d, d, 16);
                }
            } else if (MODE == 0) {
                wa[r][0] = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(Wr, (u32)lane << 4, (u32)(I * nch_all + c) << 10, 2));
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int k0 = 256 * c + 64 * j + 16 * lg;
                    const u32 off = k0 < K ? (u32)(16 * I + lr) * (u32)K + (u32)k0 : RSRC_OOB;
                    wa[r][j] = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(Wr, off, 0, 2));
                }
            }
        }
        if (PL) return;                                                   // activations: loadB after the prologue
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int t = DOT ? 0 : 16 * b + lr, k = 256 * c + 64 * j + 16 * lg;   // DOT: every lane token 0
                const bool in = t < M && k < K;
                if (QL == QL_WORDS) {                                     // 4 words (k / 4 + i, t): 16 lanes read 64 bytes
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        B[j][b][i] = (int)__builtin_amdgcn_raw_buffer_load_b32(Q, in ? ((u32)((k >> 2) + i) * (u32)ldq + (u32)t) << 2 : RSRC_OOB, 0, 0);
                } else {
                    const u32 off = in ? (QL == QL_BLOCKS ? (u32)tb_offset(t, k, K) : (u32)t * (u32)K + (u32)k) : RSRC_OOB;
                    B[j][b] = __builtin_bit_cast(int4v, __builtin_amdgcn_raw_buffer_load_b128(Q, off, 0, 0));
                }
            }
    };

    int4v acc[TR][NB];
    int dacc[TR][2];                                                      // DOT: row lr, k-block lg, two chains
#pragma unroll
    for (int r = 0; r < TR; ++r) {
        dacc[r][0] = dacc[r][1] = 0;
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[r][b] = int4v{0, 0, 0, 0};
    }
    // without a prologue, the codebook's entries are loaded first (fill_table_i8's split, entry tid + blockDim j), so the
    // table fill waits for them alone while the words and activations are still on their way
    constexpr int TE = 4;
    u32 t8w[TE];
    const bool early = MODE == 0 && !PL && blockDim.x >= 1024 / TE;     // uniform
    const i8* t8p = S.t8 + (S.rows_per_table > 0 ? (size_t)(16 * I0 / S.rows_per_table) * 1024 : 0);
    if (early) {
#pragma unroll
        for (int j = 0; j < TE; ++j) {
            const int e = (int)threadIdx.x + (int)blockDim.x * j;
            if (e < 1024) t8w[j] = gptr((const u16*)t8p)[e & 511];
        }
    }
    if (!PL && c0 + wave < nch) load(c0 + wave);
    if (OVS && pw >= 0 && c0 + pw < nch) load(c0 + pw);
    // epilogue scales, loaded with the operands (wave 0 stores; OVS: wave 8)
    float4_t rsv[TR];
    float sv[NB];
#pragma unroll
    for (int r = 0; r < TR; ++r) rsv[r] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < NB; ++b) sv[b] = 0.f;
    if (ODT != TCQ_I32 && pw == 0) {
#pragma unroll
        for (int r = 0; r < TR; ++r) rsv[r] = gptr((const float4_t*)(S.rs + 16 * min(I0 + r, tiles_m - 1) + 4 * lg))[0];
        if constexpr (!PL) {
#pragma unroll
            for (int b = 0; b < NB; ++b) sv[b] = gptr(s)[min(16 * b + lr, M - 1)];
        }
    }
    // the A fragment of packed word hi (16 weights of this lane's row, looked up in the table)
    auto frag = [&](u32 hi) {
        const u32 hn = (u32)__builtin_amdgcn_mov_dpp((int)hi, 0x12F, 0xf, 0xf, false);
        u32 e0[4], e1[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const u32 x = pk_code(p == 0 ? hi : __builtin_amdgcn_alignbit(hi, hn, 32 - 4 * p));
            e0[p] = *(const u16*)((const char*)tab + (((x >> 22) << ESH) | cp4));             // pair p
            e1[p] = *(const u16*)((const char*)tab + ((((x >> 6) & 1023u) << ESH) | cp4));    // pair p + 4
        }
        return int4v{(int)(e0[0] | (e0[1] << 16)), (int)(e0[2] | (e0[3] << 16)), (int)(e1[0] | (e1[1] << 16)),
                     (int)(e1[2] | (e1[3] << 16))};
    };
    if constexpr (OVS) {
        constexpr int SY = PL == PRO_LAYER ? WAVES_SYNCS : WAVES_SYNCS / 2;   // the prologue's barriers
        const bool on = pw >= 0 && c0 + pw < nch;                         // uniform
        int4v Af[4];
        if (pw < 0) {                                                     // the prologue waves
            run_prologue<PL, 8>(P, pro, [] {});
        } else {                                                          // the table, then the fragments, beside the prologue
            const i8* t8 = S.t8 + (S.rows_per_table > 0 ? (size_t)(16 * I0 / S.rows_per_table) * 1024 : 0);
            for (int e = (int)threadIdx.x - 512; e < 1024; e += 64 * npw) {
                const int h = e & 511;
                int v0 = gptr(t8)[2 * h];
                const int v1 = gptr(t8)[2 * h + 1];
                if (e >> 9) v0 = -v0;
                const u32 v = (u32)(v0 & 0xff) | ((u32)(v1 & 0xff) << 8);
                const u32 vv = v | (v << 16);
#pragma unroll
                for (int cc = 0; cc < SM_C; cc += 4) *(uint4_t*)(tab + e * SM_C + cc) = uint4_t{vv, vv, vv, vv};
            }
#pragma unroll
            for (int i = 0; i < SY; ++i) {
                __syncthreads();
                if (i == 0 && on) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) Af[j] = frag(wa[0][0][j]);
                }
            }
        }
        __syncthreads();                                                  // the row is in pro.qs
        if (pw == 0) sv[0] = pro.sc;
        if (on) {
            loadB(c0 + pw);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[0][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(Af[j], B[j][0], acc[0][0], 0, 0, 0);
        }
    } else {
        if (early) {
#pragma unroll
            for (int j = 0; j < TE; ++j) {
                const int e = (int)threadIdx.x + (int)blockDim.x * j;
                if (e < 1024) {                                            // fill_table_i8's entry e from its loaded pair
                    int v0 = (int)(i8)(t8w[j] & 0xff);
                    const int v1 = (int)(i8)(t8w[j] >> 8);
                    if (e >> 9) v0 = -v0;
                    const u32 v = (u32)(v0 & 0xff) | ((u32)(v1 & 0xff) << 8);
                    const u32 vv = v | (v << 16);
#pragma unroll
                    for (int c = 0; c < SM_C; c += 4) *(uint4_t*)(tab + e * SM_C + c) = uint4_t{vv, vv, vv, vv};
                }
            }
        } else if (MODE == 0) {
            fill_table_i8(tab, t8p);
        }
        if constexpr (PL > 0) run_prologue<PL, PL == PRO_PRE ? 0 : 8>(P, pro, [&] {
            if (c0 + wave < nch) load(c0 + wave);
        });
        __syncthreads();
        if constexpr (PL > 0) {
            sv[0] = pro.sc;
            if (c0 + wave < nch) loadB(c0 + wave);
        }
        for (int c = c0 + wave; c < nch; c += nw) {
            if (c != c0 + wave) {
                load(c);
                if constexpr (PL > 0) loadB(c);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int r = 0; r < TR; ++r) {
                    int4v A;
                    if (MODE == 0) {
                        A = frag(wa[r][0][j]);
                    } else {
                        A = __builtin_bit_cast(int4v, wa[r][j]);
                    }
                    if constexpr (DOT) {
                        dacc[r][j & 1] = dot_product(A, B[j][0], dacc[r][j & 1]);
                    } else {
#pragma unroll
                        for (int b = 0; b < NB; ++b) acc[r][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B[j][b], acc[r][b], 0, 0, 0);
                    }
                }
            }
        }
    }
    if constexpr (DOT) {
#pragma unroll
        for (int r = 0; r < TR; ++r) acc[r][0] = dot_to_mfma_layout(dacc[r][0] + dacc[r][1], lane);
    }
    // sum the waves' partial accumulators (exact int32) through LDS, then scale and store
    if (pw > 0) {
#pragma unroll
        for (int r = 0; r < TR; ++r)
#pragma unroll
            for (int b = 0; b < NB; ++b) red[(((pw - 1) * TR + r) * NB + b) * 64 + lane] = acc[r][b];
    }
    __syncthreads();
    if (pw != 0) return;
    for (int w = 0; w < npw - 1; ++w)
#pragma unroll
        for (int r = 0; r < TR; ++r)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[r][b] += red[((w * TR + r) * NB + b) * 64 + lane];
#pragma unroll
    for (int r = 0; r < TR; ++r) {
        const int I = I0 + r;
        if (I >= tiles_m) break;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int t = 16 * b + lr;
            if (t < M) {
                const size_t o = (size_t)t * ldz + 16 * I + 4 * lg;
                if (ODT == TCQ_I32) {
                    *gptr((int4v*)((int*)S.out + (KS > 1 ? (size_t)blockIdx.z * M * ldz : 0) + o)) = acc[r][b];
                } else {
                    const float st = sv[b];
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = ((float)acc[r][b][e] * st) * rsv[r][e];
                    if (ODT == TCQ_F32) {
                        *gptr((float4_t*)((float*)S.out + o)) = float4_t{v[0], v[1], v[2], v[3]};
                    } else {
                        const u32 lo = bf16x2(v[0], v[1]);
                        const u32 hi = bf16x2(v[2], v[3]);
                        *gptr((u64*)((u16*)S.out + o)) = (u64)lo | ((u64)hi << 32);
                    }
                }
            }
        }
    }
}

// Streaming plan of the fused decode for one token block (M <= 16) and large layers (the backbone's gate/up and down
// products at one token: 8.5 and 8.3 us on MI355X against 10.0 and 10.4 on the workgroup plan): a workgroup takes
// RPW = NW / WPR tile rows, WPR waves per tile row, and wave p of a row takes its chunks p, p + WPR, ... (at most CMAX).
// Every chunk's words are loaded at entry (they come from HBM); the activation fragments (L2-resident) one chunk ahead.
// The table has 16 copies (lane l reads copy l mod 16: two lanes per copy in a half-wave), filled once per workgroup. The
// WPR partial sums of a row are added through LDS, over the table, once every wave has finished its lookups (exact int32).
constexpr int GV_C = 16;
constexpr int GV_CMAX = 8;
constexpr int GV_NW = 16;              // waves per workgroup (one 64 KiB table fill per 16 waves)

// LO (TCQ_Z_W128T, FP32 scaled z, RPW = 8): the workgroup's 128 rows are one 128-row block of the segment; the first seven
// stages of the block Walsh of the whole segment (h = 1 .. 64, which stay inside such a block) run here, in the reference's
// stage order, and the block is stored transposed: zt[(t * 128 + o) * (m / 128) + blk] for row 128 blk + o of token t.
// DOT (M == 1): the product on v_dot4c_i32_i8 (dot_product) instead of the MFMA; the epilogues are shared.
// PL > 0: activations from the prologue, as k_gemm_small.
// OV (the layer prologue of a 2048-wide row): the prologue runs on waves 0 .. 3 from entry (panp_waves,
// waves_rotate_quantize, at a raised issue priority) while the other waves fill the table and then decode the weight
// fragments of their chunks into registers, one chunk after each of the prologue's WAVES_SYNCS barriers (the first of
// which is also the table's); one more barrier hands the row to every wave for its products. The same row, sums and
// outputs as without OV.
template <int ODT, bool QB, int WPR, int NW, int KS = 1, bool LO = false, bool DOT = false, int PL = 0, bool OV = false>
__global__ __launch_bounds__(64 * NW) void k_gemv_tcq(const typename PackOf<PL>::type P, const i8* q, const float* s, int M, int K,
                                                      int ldz) {
    static_assert(KS == 1 || ODT == TCQ_I32, "K parts are int32 sums");
    static_assert(PL == 0 || (!QB && !DOT), "prologue: one token");
    static_assert(!OV || (PL == PRO_LAYER && !DOT && NW >= 4), "overlapped prologue: the layer prologue on four waves");
    __shared__ ProLds<PL ? PL : PRO_LAYER> pro;
    __shared__ WavesLds qd[1];                                            // OV only
    static_assert(!LO || (ODT == TCQ_F32 && KS == 1 && NW / WPR == 8), "stage-split output: FP32 z, 8 tile rows per workgroup");
    constexpr int RPW = NW / WPR;
    __shared__ __attribute__((aligned(16))) u32 tab[1024 * GV_C];
    const tcq_gemm_seg S = P.s[blockIdx.y];
    const int tiles_m = S.m >> 4, nch_all = (K + 255) >> 8;
    const int c0 = KS > 1 ? (int)blockIdx.z * ((nch_all + KS - 1) / KS) : 0;
    const int nch = KS > 1 ? min(nch_all, c0 + (nch_all + KS - 1) / KS) : nch_all;   // chunks c0 .. nch - 1 (K part z)
    const int I0 = blockIdx.x * RPW;
    if (I0 >= tiles_m) return;                                            // uniform
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int slot = wave / WPR, part = wave % WPR;
    const int I = min(I0 + slot, tiles_m - 1);                            // a row past the end decodes the last (never stored)
    const int lr = lane & 15, lg = lane >> 4;
    const u32 cp4 = (u32)(lane & (GV_C - 1)) << 2;
    const rsrc_t Wr = make_rsrc(S.w, (u32)(tiles_m * nch_all) << 10);
    const rsrc_t Q = make_rsrc(q, QB ? 16u * (u32)K : (u32)M * (u32)K);
    constexpr int CM = PL ? (((1 << ProShape<PL ? PL : PRO_LAYER>::L) / 256 + KS - 1) / KS + WPR - 1) / WPR : GV_CMAX;   // chunks per wave
    uint4_t wa[CM];
    auto loadW = [&] {
#pragma unroll
        for (int i = 0; i < CM; ++i) {
            const int c = c0 + part + WPR * i;
            if (c < nch) wa[i] = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(Wr, (u32)lane << 4, (u32)(I * nch_all + c) << 10, 2));
        }
    };
    // the codebook's entries first (the table fill's split: entry tid - t0 + (64 NW - t0) j, t0 = the first filling thread:
    // 0, or 256 past the four prologue waves with OV), so the fill waits for them alone
    constexpr int FT0 = OV ? 256 : 0;
    static_assert(2 * (64 * NW - FT0) >= 1024, "two table entries per filling thread");
    u32 t8w[2];
    const i8* t8p = S.t8 + (S.rows_per_table > 0 ? (size_t)(16 * I0 / S.rows_per_table) * 1024 : 0);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int e = (int)threadIdx.x - FT0 + (64 * NW - FT0) * j;
        if (e >= 0 && e < 1024) t8w[j] = gptr((const u16*)t8p)[e & 511];
    }
    if constexpr (!PL || OV) loadW();
    auto loadB = [&](int c, int4v* B) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = 256 * c + 64 * j + 16 * lg, t = DOT ? 0 : lr;              // DOT: every lane token 0
            if constexpr (PL > 0) {                                        // the prologue's row (LDS)
                B[j] = (t < M && k < K) ? *(const int4v*)((const char*)pro.qs + k) : int4v{0, 0, 0, 0};
            } else {
                const u32 off = (t < M && k < K) ? (QB ? (u32)tb_offset(t, k, K) : (u32)t * (u32)K + (u32)k) : RSRC_OOB;
                B[j] = __builtin_bit_cast(int4v, __builtin_amdgcn_raw_buffer_load_b128(Q, off, 0, 0));
            }
        }
    };
    int4v Bf[2][4];                                                        // activation fragments, two chunks in turn
    if constexpr (!PL) loadB(c0 + part, Bf[0]);
    float4_t rsv = float4_t{0.f, 0.f, 0.f, 0.f};
    float sv = 0.f;
    if (ODT != TCQ_I32 && part == 0) {
        rsv = gptr((const float4_t*)(S.rs + 16 * I + 4 * lg))[0];
        if constexpr (!PL) sv = gptr(s)[min(lr, M - 1)];
    }
    // the table, filled by threads from t0 on (OV: the decode waves alone; the prologue waves start at once)
    auto fill_table = [&](int t0) {                                        // t0 = FT0: from the loaded pairs
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int e = (int)threadIdx.x - t0 + (64 * NW - t0) * j;
            if (e < 0 || e >= 1024) continue;
            int v0 = (int)(i8)(t8w[j] & 0xff);
            const int v1 = (int)(i8)(t8w[j] >> 8);
            if (e >> 9) v0 = -v0;
            const u32 v = (u32)(v0 & 0xff) | ((u32)(v1 & 0xff) << 8);
            const u32 vv = v | (v << 16);
#pragma unroll
            for (int c = 0; c < GV_C; c += 4) *(uint4_t*)(tab + e * GV_C + c) = uint4_t{vv, vv, vv, vv};
        }
    };
    if constexpr (!OV) {
        fill_table(0);
        if constexpr (PL > 0) run_prologue<PL>(P, pro, loadW);
        __syncthreads();
    }
    // the A fragment of one packed word: 16 weights of this lane's row, looked up in the table
    auto frag = [&](u32 hi) {
        const u32 hn = (u32)__builtin_amdgcn_mov_dpp((int)hi, 0x12F, 0xf, 0xf, false);
        u16x2_t a[4];                                                      // pairs p (a[0], a[1]) and p + 4 (a[2], a[3])
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const u32 x = pk_code(p == 0 ? hi : __builtin_amdgcn_alignbit(hi, hn, 32 - 4 * p));
            a[p >> 1][p & 1] = *(const u16*)((const char*)tab + (((x >> 22) << 6) | cp4));
            a[2 + (p >> 1)][p & 1] = *(const u16*)((const char*)tab + ((x & 0xFFC0u) | cp4));
        }
        return int4v{__builtin_bit_cast(int, a[0]), __builtin_bit_cast(int, a[1]), __builtin_bit_cast(int, a[2]),
                     __builtin_bit_cast(int, a[3])};
    };
    int4v acc = int4v{0, 0, 0, 0};
    int dacc[2] = {0, 0};                                                  // DOT: row lr, k-block lg, two chains
    if constexpr (OV) {
        int4v Af[CM][4];
        auto decode = [&](int i) {
            if (c0 + part + WPR * i < nch) {                               // uniform
#pragma unroll
                for (int j = 0; j < 4; ++j) Af[i][j] = frag(wa[i][j]);
            }
        };
        if (wave < 4) {                                                    // uniform: the prologue waves
            const bool store = blockIdx.x == 0 && blockIdx.y == 0;
            const auto bar = [] { __syncthreads(); };
            float v[8];
            __builtin_amdgcn_s_setprio(2);
            panp_waves<TCQ_I32, 4>(P.a, 0, store, v, qd[0], NoMid{}, bar);
            waves_rotate_quantize<4>(v, qd[0], pro.qs, &pro.sc, store ? P.q : nullptr, store ? P.scale : nullptr, bar);
            __builtin_amdgcn_s_setprio(0);
#pragma unroll
            for (int i = 0; i < CM; ++i) decode(i);
        } else {                                                           // the others: the table, then a chunk per barrier
            fill_table(256);
#pragma unroll
            for (int i = 0; i < (CM > WAVES_SYNCS ? CM : WAVES_SYNCS); ++i) {
                if (i < WAVES_SYNCS) __syncthreads();
                if (i < CM) decode(i);
            }
        }
        __syncthreads();                                                   // the row is in pro.qs
        if (ODT != TCQ_I32 && part == 0) sv = pro.sc;
#pragma unroll
        for (int i = 0; i < CM; ++i) {
            const int c = c0 + part + WPR * i;
            if (c >= nch) continue;                                        // uniform
            loadB(c, Bf[0]);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(Af[i][j], Bf[0][j], acc, 0, 0, 0);
        }
    } else {
        if constexpr (PL > 0) {
            if (ODT != TCQ_I32 && part == 0) sv = pro.sc;
            loadB(c0 + part, Bf[0]);
        }
#pragma unroll
        for (int i = 0; i < CM; ++i) {
            const int c = c0 + part + WPR * i;
            if (c >= nch) continue;                                        // uniform
            if (i + 1 < CM && c + WPR < nch) loadB(c + WPR, Bf[(i + 1) & 1]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int4v A = frag(wa[i][j]);
                if constexpr (DOT) dacc[j & 1] = dot_product(A, Bf[i & 1][j], dacc[j & 1]);
                else acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, Bf[i & 1][j], acc, 0, 0, 0);
            }
        }
    }
    if constexpr (DOT) acc = dot_to_mfma_layout(dacc[0] + dacc[1], lane);
    if constexpr (WPR > 1) {
        int4v* red = (int4v*)tab;                                          // the table is dead once every wave is past here
        __syncthreads();
        if (part > 0) red[((slot * (WPR - 1)) + part - 1) * 64 + lane] = acc;
        __syncthreads();
        if (part != 0 && !LO) return;
        if (part == 0) {
#pragma unroll
            for (int w = 0; w < WPR - 1; ++w) acc += red[(slot * (WPR - 1) + w) * 64 + lane];
        }
    }
    if constexpr (LO) {                                                    // every wave reaches the barrier below
        float* zb = (float*)tab + 4096;                                    // past the reduction slots: M rows of 128
        if (part == 0) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = ((float)acc[e] * sv) * rsv[e];
            float a = v[0], b = v[1];                                      // h = 1, 2: row pairs in the lane's 4 rows
            v[0] = a + b; v[1] = a - b;
            a = v[2]; b = v[3];
            v[2] = a + b; v[3] = a - b;
            a = v[0]; b = v[2];
            v[0] = a + b; v[2] = a - b;
            a = v[1]; b = v[3];
            v[1] = a + b; v[3] = a - b;
#pragma unroll
            for (int m = 16; m <= 32; m *= 2)                              // h = 4, 8: rows 4 lg + e, lanes 16 lg + lr
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float pv = lane_xor(v[e], m, lane);
                    v[e] = (lane & m) ? pv - v[e] : v[e] + pv;
                }
            if (lr < M) {
#pragma unroll
                for (int e = 0; e < 4; ++e) zb[lr * 128 + 16 * slot + 4 * lg + e] = v[e];
            }
        }
        __syncthreads();
        if (wave < M) {                                                    // h = 16, 32, 64: token `wave`, rows l and l + 64
            float a = zb[wave * 128 + lane], b = zb[wave * 128 + 64 + lane];
#pragma unroll
            for (int m = 16; m <= 32; m *= 2) {
                const float pa = lane_xor(a, m, lane), pb = lane_xor(b, m, lane);
                a = (lane & m) ? pa - a : a + pa;
                b = (lane & m) ? pb - b : b + pb;
            }
            const float x = a;
            a = x + b;
            b = x - b;
            const int nb = S.m >> 7, blk = I0 >> 3;
            float* zt = (float*)S.out + (size_t)wave * 128 * nb;
            gptr(zt)[(size_t)lane * nb + blk] = a;
            gptr(zt)[(size_t)(lane + 64) * nb + blk] = b;
        }
        return;
    }
    if (I0 + slot >= tiles_m) return;
    const int t = lr;
    if (t >= M) return;
    const size_t o = (size_t)t * ldz + 16 * I + 4 * lg;
    if (ODT == TCQ_I32) {
        *gptr((int4v*)((int*)S.out + (KS > 1 ? (size_t)blockIdx.z * M * ldz : 0) + o)) = acc;
    } else {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = ((float)acc[e] * sv) * rsv[e];
        if (ODT == TCQ_F32) {
            *gptr((float4_t*)((float*)S.out + o)) = float4_t{v[0], v[1], v[2], v[3]};
        } else {
            const u32 lo = bf16x2(v[0], v[1]);
            const u32 hi = bf16x2(v[2], v[3]);
            *gptr((u64*)((u16*)S.out + o)) = (u64)lo | ((u64)hi << 32);
        }
    }
}

// =========================================================================================================== C ABI
template <int MODE, int NB, int TR, int QL, bool RB, bool DOT = false>
static void launch_small_nb(dim3 grid, dim3 block, hipStream_t st, const SegPack& P, const i8* q, const float* s, int M, int K,
                            int ldo, int ldq, int odt) {
    switch (odt) {
        case TCQ_F32: launch_k(k_gemm_small<MODE, NB, TCQ_F32, TR, QL, RB, 1, DOT>, grid, block, 0, st, P, q, s, M, K, ldo, ldq); break;
        case TCQ_BF16: launch_k(k_gemm_small<MODE, NB, TCQ_BF16, TR, QL, RB, 1, DOT>, grid, block, 0, st, P, q, s, M, K, ldo, ldq); break;
        default: launch_k(k_gemm_small<MODE, NB, TCQ_I32, TR, QL, RB, 1, DOT>, grid, block, 0, st, P, q, s, M, K, ldo, ldq); break;
    }
}
template <int MODE, int TR, int QL, bool RB = false>
static void launch_small_qb(dim3 grid, dim3 block, hipStream_t st, const SegPack& P, const i8* q, const float* s, int M, int K,
                            int ldo, int ldq, int odt) {
    if (M <= 16) launch_small_nb<MODE, 1, TR, QL, RB>(grid, block, st, P, q, s, M, K, ldo, ldq, odt);
    else if (M <= 32) launch_small_nb<MODE, 2, TR, QL, RB>(grid, block, st, P, q, s, M, K, ldo, ldq, odt);
    else launch_small_nb<MODE, 4, TR, QL, RB>(grid, block, st, P, q, s, M, K, ldo, ldq, odt);
}
template <int MODE, int TR>
static void launch_small_tr(dim3 grid, dim3 block, hipStream_t st, const SegPack& P, const i8* q, const float* s, int M, int K,
                            int ldo, int odt, bool qb, bool dot) {
    if (dot && qb) launch_small_nb<MODE, 1, TR, QL_BLOCKS, false, true>(grid, block, st, P, q, s, M, K, ldo, 0, odt);
    else if (dot) launch_small_nb<MODE, 1, TR, QL_ROWS, false, true>(grid, block, st, P, q, s, M, K, ldo, 0, odt);
    else if (qb) launch_small_qb<MODE, TR, QL_BLOCKS>(grid, block, st, P, q, s, M, K, ldo, 0, odt);
    else launch_small_qb<MODE, TR, QL_ROWS>(grid, block, st, P, q, s, M, K, ldo, 0, odt);
}

template <int ODT, bool QB, bool DOT>
static void launch_gv(int wpr, int rows, int nseg, hipStream_t st, const SegPack& P, const i8* q, const float* s, int M, int K,
                      int ldo) {
    const int rpw = GV_NW / wpr;
    const dim3 grid((rows + rpw - 1) / rpw, nseg), block(64 * GV_NW);
    switch (wpr) {
        case 1: launch_k(k_gemv_tcq<ODT, QB, 1, GV_NW, 1, false, DOT>, grid, block, 0, st, P, q, s, M, K, ldo); break;
        case 2: launch_k(k_gemv_tcq<ODT, QB, 2, GV_NW, 1, false, DOT>, grid, block, 0, st, P, q, s, M, K, ldo); break;
        case 4: launch_k(k_gemv_tcq<ODT, QB, 4, GV_NW, 1, false, DOT>, grid, block, 0, st, P, q, s, M, K, ldo); break;
        case 8: launch_k(k_gemv_tcq<ODT, QB, 8, GV_NW, 1, false, DOT>, grid, block, 0, st, P, q, s, M, K, ldo); break;
        default: launch_k(k_gemv_tcq<ODT, QB, 16, GV_NW, 1, false, DOT>, grid, block, 0, st, P, q, s, M, K, ldo); break;
    }
}

// K parts (int32 sums only): grid.z = KS parts
template <int MODE, int KS, int QL, bool DOT>
static void launch_small_parts(dim3 grid, dim3 block, hipStream_t st, const SegPack& P, const i8* q, const float* s, int M, int K,
                               int ldo) {
    if (DOT || M <= 16) launch_k(k_gemm_small<MODE, 1, TCQ_I32, 1, QL, false, KS, DOT>, grid, block, 0, st, P, q, s, M, K, ldo, 0);
    else if (M <= 32) launch_k(k_gemm_small<MODE, 2, TCQ_I32, 1, QL, false, KS>, grid, block, 0, st, P, q, s, M, K, ldo, 0);
    else launch_k(k_gemm_small<MODE, 4, TCQ_I32, 1, QL, false, KS>, grid, block, 0, st, P, q, s, M, K, ldo, 0);
}
template <bool QB, int KS, bool DOT>
static void launch_gv_parts(int wpr, int rows, int nseg, hipStream_t st, const SegPack& P, const i8* q, const float* s, int M, int K,
                            int ldo) {
    const int rpw = GV_NW / wpr;
    const dim3 grid((rows + rpw - 1) / rpw, nseg, KS), block(64 * GV_NW);
    switch (wpr) {
        case 1: launch_k(k_gemv_tcq<TCQ_I32, QB, 1, GV_NW, KS, false, DOT>, grid, block, 0, st, P, q, s, M, K, ldo); break;
        case 2: launch_k(k_gemv_tcq<TCQ_I32, QB, 2, GV_NW, KS, false, DOT>, grid, block, 0, st, P, q, s, M, K, ldo); break;
        case 4: launch_k(k_gemv_tcq<TCQ_I32, QB, 4, GV_NW, KS, false, DOT>, grid, block, 0, st, P, q, s, M, K, ldo); break;
        case 8: launch_k(k_gemv_tcq<TCQ_I32, QB, 8, GV_NW, KS, false, DOT>, grid, block, 0, st, P, q, s, M, K, ldo); break;
        default: launch_k(k_gemv_tcq<TCQ_I32, QB, 16, GV_NW, KS, false, DOT>, grid, block, 0, st, P, q, s, M, K, ldo); break;
    }
}
template <int MODE, int KS, bool DOT>
static void launch_parts(bool qb, int wpr, int rows, int nseg, int nw, hipStream_t st, const SegPack& P, const i8* q, const float* s,
                         int M, int K, int ldo) {
    if (MODE == 0 && wpr > 0) {
        if (qb) launch_gv_parts<true, KS, DOT>(wpr, rows, nseg, st, P, q, s, M, K, ldo);
        else launch_gv_parts<false, KS, DOT>(wpr, rows, nseg, st, P, q, s, M, K, ldo);
        return;
    }
    const dim3 grid(rows, nseg, KS), block(64 * nw);
    if (qb) launch_small_parts<MODE, KS, QL_BLOCKS, DOT>(grid, block, st, P, q, s, M, K, ldo);
    else launch_small_parts<MODE, KS, QL_ROWS, DOT>(grid, block, st, P, q, s, M, K, ldo);
}
template <int MODE, int KS>
static void launch_parts_dot(bool dot, bool qb, int wpr, int rows, int nseg, int nw, hipStream_t st, const SegPack& P, const i8* q,
                             const float* s, int M, int K, int ldo) {
    if (dot) launch_parts<MODE, KS, true>(qb, wpr, rows, nseg, nw, st, P, q, s, M, K, ldo);
    else launch_parts<MODE, KS, false>(qb, wpr, rows, nseg, nw, st, P, q, s, M, K, ldo);
}

template <bool QB, bool DOT>
static void launch_gv_odt(int odt, int wpr, int rows, int nseg, hipStream_t st, const SegPack& P, const i8* q, const float* s,
                          int M, int K, int ldo) {
    switch (odt) {
        case TCQ_F32: launch_gv<TCQ_F32, QB, DOT>(wpr, rows, nseg, st, P, q, s, M, K, ldo); break;
        case TCQ_BF16: launch_gv<TCQ_BF16, QB, DOT>(wpr, rows, nseg, st, P, q, s, M, K, ldo); break;
        default: launch_gv<TCQ_I32, QB, DOT>(wpr, rows, nseg, st, P, q, s, M, K, ldo); break;
    }
}

// Waves per tile row of the streaming plan for a fused decode of `tiles` tile rows (all segments) of nch chunks, or 0 when
// the workgroup plan serves it: at most GV_CMAX chunks per wave, and enough waves to cover the chip (4096) where the rows
// allow; row-group tables must hold whole workgroups.
static int gv_waves_per_row(const tcq_gemm_seg* segs, int nseg, int M, int nch, int tiles) {
    if (M > 16 || (size_t)tiles * nch < 4096 || nch > 16 * GV_CMAX) return 0;
    int wpr = 1;
    while (wpr < 16 && (wpr * GV_CMAX < nch || tiles * wpr < 4096)) wpr *= 2;
    while (wpr > 1 && (wpr / 2) >= nch) wpr /= 2;
    const int rpw = GV_NW / wpr;
    for (int i = 0; i < nseg; ++i)
        if (segs[i].rows_per_table > 0 && (segs[i].rows_per_table / 16) % rpw) return 0;
    return wpr;
}

template <int MODE>
static int gemm_small(const tcq_gemm_seg* segs, int nseg, const int8_t* q, const float* s, int M, int K, int odt, int ldo,
                      tcq_stream_t stream) {
    if (!segs || !q || nseg <= 0 || M <= 0 || K <= 0 || ldo <= 0) return TCQ_ERR_ARG;
    const bool qb = odt & TCQ_Q_TOKEN_BLOCKS;                          // q in the token-block layout
    if ((odt & TCQ_K_PARTS2) && (odt & TCQ_K_PARTS4)) return TCQ_ERR_ARG;
    const int parts = (odt & TCQ_K_PARTS4) ? 4 : (odt & TCQ_K_PARTS2) ? 2 : 1;
    const bool w128 = odt & TCQ_Z_W128T, dot = odt & TCQ_DOT4;
    odt &= ~(TCQ_Q_TOKEN_BLOCKS | TCQ_K_PARTS2 | TCQ_K_PARTS4 | TCQ_Z_W128T | TCQ_DOT4);
    if (w128 && (MODE != 0 || odt != TCQ_F32 || parts > 1 || M > 16 || K > 256 * 2 * GV_CMAX)) return TCQ_ERR_UNSUPPORTED;
    if (dot && M != 1) return TCQ_ERR_UNSUPPORTED;
    if (odt != TCQ_F32 && odt != TCQ_BF16 && odt != TCQ_I32) return TCQ_ERR_DTYPE;
    if (parts > 1 && odt != TCQ_I32) return TCQ_ERR_DTYPE;
    if (odt != TCQ_I32 && !s) return TCQ_ERR_ARG;
    if (nseg > TCQ_MAX_SEGS || M > 64) return TCQ_ERR_UNSUPPORTED;
    if (K % 16) return TCQ_ERR_SHAPE;
    if (ldo % 4 || (uintptr_t)q % 16) return TCQ_ERR_ALIGN;
    SegPack P = {};
    int max_m = 0;
    for (int i = 0; i < nseg; ++i) {
        const tcq_gemm_seg& g = segs[i];
        if (!g.w || !g.out || (MODE == 0 && !g.t8) || (odt != TCQ_I32 && !g.rs) || g.m <= 0) return TCQ_ERR_ARG;
        if (g.m % 16) return TCQ_ERR_SHAPE;
        if (g.rows_per_table < 0 || (g.rows_per_table > 0 && (g.rows_per_table % 16 || g.m % g.rows_per_table))) return TCQ_ERR_SHAPE;
        if ((size_t)g.m * K >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
        const size_t osz = odt == TCQ_BF16 ? 2 : 4;
        if ((uintptr_t)g.out % (4 * osz) || (g.rs && (uintptr_t)g.rs % 16)) return TCQ_ERR_ALIGN;
        P.s[i] = g;
        if (g.m > max_m) max_m = g.m;
    }
    if ((size_t)M * K >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
    if (parts > 1 && (size_t)parts * M * ldo >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
    const int nch = (K + 255) / 256, nw = nch < SM_MAXW ? nch : SM_MAXW;
    hipStream_t st = (hipStream_t)stream;
    const i8* qq = (const i8*)q;
    if (w128) {                                        // stage-split gated-MLP input: the streaming plan, 8 tile rows per workgroup
        for (int i = 0; i < nseg; ++i)
            if (segs[i].m % 128 || (segs[i].rows_per_table > 0 && segs[i].rows_per_table % 128)) return TCQ_ERR_SHAPE;
        const dim3 grid(max_m / 128, nseg), block(64 * GV_NW);
        if (dot && qb) launch_k(k_gemv_tcq<TCQ_F32, true, 2, GV_NW, 1, true, true>, grid, block, 0, st, P, qq, s, M, K, ldo);
        else if (dot) launch_k(k_gemv_tcq<TCQ_F32, false, 2, GV_NW, 1, true, true>, grid, block, 0, st, P, qq, s, M, K, ldo);
        else if (qb) launch_k(k_gemv_tcq<TCQ_F32, true, 2, GV_NW, 1, true>, grid, block, 0, st, P, qq, s, M, K, ldo);
        else launch_k(k_gemv_tcq<TCQ_F32, false, 2, GV_NW, 1, true>, grid, block, 0, st, P, qq, s, M, K, ldo);
        return launch_status();
    }
    if (parts > 1) {                                   // K parts: each part a product over its chunks, int32 out
        const int nchp = (nch + parts - 1) / parts, nwp = nchp < SM_MAXW ? nchp : SM_MAXW;
        int tiles = 0;
        for (int i = 0; i < nseg; ++i) tiles += segs[i].m / 16;
        const int wpr = MODE == 0 ? gv_waves_per_row(segs, nseg, M, nchp, tiles * parts) : 0;
        if (parts == 2) launch_parts_dot<MODE, 2>(dot, qb, wpr, max_m / 16, nseg, nwp, st, P, qq, s, M, K, ldo);
        else launch_parts_dot<MODE, 4>(dot, qb, wpr, max_m / 16, nseg, nwp, st, P, qq, s, M, K, ldo);
        return launch_status();
    }
    // two tile rows per workgroup when there are many (their activation fragments are then loaded once for both), at most 8
    // waves (the partial sums of both rows fit the LDS) and row-group tables that never split a pair
    int tiles = 0;
    bool pairs = nw <= 8;
    for (int i = 0; i < nseg; ++i) {
        tiles += segs[i].m / 16;
        if (segs[i].rows_per_table > 0 && (segs[i].rows_per_table / 16) % 2) pairs = false;
    }
    pairs = pairs && tiles >= 384;
    if (MODE == 0) {
        const int wpr = gv_waves_per_row(segs, nseg, M, nch, tiles);
        if (wpr > 0) {
            if (dot && qb) launch_gv_odt<true, true>(odt, wpr, max_m / 16, nseg, st, P, qq, s, M, K, ldo);
            else if (dot) launch_gv_odt<false, true>(odt, wpr, max_m / 16, nseg, st, P, qq, s, M, K, ldo);
            else if (qb) launch_gv_odt<true, false>(odt, wpr, max_m / 16, nseg, st, P, qq, s, M, K, ldo);
            else launch_gv_odt<false, false>(odt, wpr, max_m / 16, nseg, st, P, qq, s, M, K, ldo);
            return launch_status();
        }
    }
    const dim3 block(64 * nw);
    if (pairs) launch_small_tr<MODE, 2>(dim3((max_m / 16 + 1) / 2, nseg), block, st, P, qq, s, M, K, ldo, odt, qb, dot);
    else launch_small_tr<MODE, 1>(dim3(max_m / 16, nseg), block, st, P, qq, s, M, K, ldo, odt, qb, dot);
    return launch_status();
}

extern "C" int tcq_gemm_tcq(const tcq_gemm_seg* segs, int nseg, const int8_t* q, const float* s, int M, int K, int out_dtype,
                            int ldo, tcq_stream_t stream) {
    return gemm_small<0>(segs, nseg, q, s, M, K, out_dtype, ldo, stream);
}

extern "C" int tcq_gemm_w8(const tcq_gemm_seg* segs, int nseg, const int8_t* q, const float* s, int M, int K, int out_dtype, int ldo,
                           tcq_stream_t stream) {
    return gemm_small<1>(segs, nseg, q, s, M, K, out_dtype, ldo, stream);
}

// ------------------------------------------------------------------------------------ products with the layer prologue
// One token: every workgroup first computes the product's INT8 row itself, on the same register + transpose engine as the
// standalone kernels and bit for bit, then its share of the product on that row (LDS); workgroup (0, 0, 0) stores the
// row's side outputs (xout, and the optional q / scale copies). Three prologues (ProShape): with acc, tcq_post_add_norm_pre's
// operations on a 2048-wide row (FP32 z out, optionally the stage-split TCQ_Z_W128T form); with part, the attention merge
// of 8 heads + rotate + quantize (int32 sums out, optionally in K parts; 8 waves, one per head); else tcq_pre's on a
// 16384-wide BF16 row x (int32 sums out, optionally in K parts). Plans as gemm_small picks them for M = 1.
static bool pal16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <int MODE, int PL, int ODT, int KS>
static void launch_pro_small(int rows, int nseg, int nw, bool pairs, hipStream_t st, const SegPackPro& P, int K, int ldo) {
    const i8* nq = nullptr;
    const float* ns = nullptr;
    if constexpr (MODE == 0 && (PL == PRO_LAYER || PL == PRO_ATTN)) {
        const int nchp = (K / 256 + KS - 1) / KS;                      // one product wave per chunk beside 8 prologue waves
        if (!pairs && nchp <= 8) {
            launch_k(k_gemm_small<MODE, 1, ODT, 1, QL_ROWS, false, KS, false, PL, true>, dim3(rows, nseg, KS), dim3(64 * (8 + nchp)), 0,
                     st, P, nq, ns, 1, K, ldo, 0);
            return;
        }
    }
    if constexpr (PL == PRO_LAYER) {
        if (pairs) {
            launch_k(k_gemm_small<MODE, 1, ODT, 2, QL_ROWS, false, KS, false, PL>, dim3((rows + 1) / 2, nseg, KS), dim3(64 * nw), 0, st,
                     P, nq, ns, 1, K, ldo, 0);
            return;
        }
    }
    launch_k(k_gemm_small<MODE, 1, ODT, 1, QL_ROWS, false, KS, false, PL>, dim3(rows, nseg, KS), dim3(64 * nw), 0, st, P, nq, ns, 1, K,
             ldo, 0);
}

template <int MODE>
static int gemm_small_pro(const tcq_gemm_seg* segs, int nseg, const tcq_prologue* pr, int K, int odt, int ldo, tcq_stream_t stream) {
    if (!segs || !pr || nseg <= 0 || ldo <= 0) return TCQ_ERR_ARG;
    if (nseg > TCQ_MAX_SEGS) return TCQ_ERR_UNSUPPORTED;
    const bool layer = pr->acc != nullptr, attn = !layer && pr->part != nullptr;   // else: rotate + quantize of x
    const bool w128 = odt & TCQ_Z_W128T;
    if ((odt & TCQ_K_PARTS2) && (odt & TCQ_K_PARTS4)) return TCQ_ERR_ARG;
    const int parts = (odt & TCQ_K_PARTS4) ? 4 : (odt & TCQ_K_PARTS2) ? 2 : 1;
    odt &= ~(TCQ_Z_W128T | TCQ_K_PARTS2 | TCQ_K_PARTS4);
    if (layer ? (K != 2048 || odt != TCQ_F32 || parts > 1 || (w128 && MODE != 0))
              : (K != (attn ? 2048 : 16384) || odt != TCQ_I32 || parts > 2 || w128))
        return TCQ_ERR_UNSUPPORTED;
    if (!pr->su || (!attn && !pr->x)) return TCQ_ERR_ARG;
    if (attn) {
        if (pr->heads != 8 || pr->chunks <= 0 || pr->chunks > MAXC || pr->keys <= 0 || pr->keys > pr->chunks * KC) return TCQ_ERR_UNSUPPORTED;
        if (!pal16(pr->part) || (uintptr_t)pr->su % 4) return TCQ_ERR_ALIGN;
    }
    int pparts = 1;
    if (layer) {
        int adt = pr->acc_dtype;
        if ((adt & TCQ_K_PARTS2) && (adt & TCQ_K_PARTS4)) return TCQ_ERR_ARG;
        pparts = (adt & TCQ_K_PARTS4) ? 4 : (adt & TCQ_K_PARTS2) ? 2 : 1;
        adt &= ~(TCQ_K_PARTS2 | TCQ_K_PARTS4);
        if (adt != TCQ_I32) return TCQ_ERR_DTYPE;
        if (!pr->s || !pr->rs || !pr->sv || !pr->xout || !pr->w || pr->col0 < 0 || pr->lda < pr->col0 + K) return TCQ_ERR_ARG;
        if (pr->bias) return TCQ_ERR_UNSUPPORTED;
        if ((size_t)pparts * pr->lda >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
        if (!pal16(pr->acc) || pr->lda % 4 || pr->col0 % 4 || !pal16(pr->rs) || !pal16(pr->sv) || !pal16(pr->xout) || !pal16(pr->w))
            return TCQ_ERR_ALIGN;
    }
    if ((!attn && (!pal16(pr->x) || !pal16(pr->su))) || (pr->q && !pal16(pr->q)) || ldo % 4) return TCQ_ERR_ALIGN;
    if (parts > 1 && (size_t)parts * ldo >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
    SegPackPro P = {};
    int max_m = 0, tiles = 0;
    for (int i = 0; i < nseg; ++i) {
        const tcq_gemm_seg& g = segs[i];
        if (!g.w || !g.out || (MODE == 0 && !g.t8) || (odt != TCQ_I32 && !g.rs) || g.m <= 0) return TCQ_ERR_ARG;
        if (g.m % 16) return TCQ_ERR_SHAPE;
        if (g.rows_per_table < 0 || (g.rows_per_table > 0 && (g.rows_per_table % 16 || g.m % g.rows_per_table))) return TCQ_ERR_SHAPE;
        if ((size_t)g.m * K >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
        if ((uintptr_t)g.out % 16 || (g.rs && (uintptr_t)g.rs % 16)) return TCQ_ERR_ALIGN;
        if (w128 && (g.m % 128 || (g.rows_per_table > 0 && g.rows_per_table % 128))) return TCQ_ERR_SHAPE;
        P.s[i] = g;
        max_m = g.m > max_m ? g.m : max_m;
        tiles += g.m / 16;
    }
    P.a = PanpArgs{pr->acc, pr->s, pr->rs, (const i8*)pr->sv, nullptr, (const u16*)pr->x, (u16*)pr->xout, (const u16*)pr->w,
                   (const i8*)pr->su, pr->lda, pr->col0, pparts, (size_t)pr->lda, pr->eps};
    P.q = (i8*)pr->q;
    P.scale = pr->scale;
    P.part = pr->part;
    P.nc = pr->chunks;
    P.keys = pr->keys;
    P.causal = pr->causal;
    P.heads = pr->heads;
    hipStream_t st = (hipStream_t)stream;
    const i8* nq = nullptr;
    const float* ns = nullptr;
    const int nch = K / 256, nchp = (nch + parts - 1) / parts, nw = nchp < SM_MAXW ? nchp : SM_MAXW;
    if (attn) {                                        // the workgroup plan on one wave per head (8), one tile row each
        if (parts == 2) launch_pro_small<MODE, PRO_ATTN, TCQ_I32, 2>(max_m / 16, nseg, AH, false, st, P, K, ldo);
        else launch_pro_small<MODE, PRO_ATTN, TCQ_I32, 1>(max_m / 16, nseg, AH, false, st, P, K, ldo);
        return launch_status();
    }
    if (layer) {
        if (w128) {
            launch_k(k_gemv_tcq<TCQ_F32, false, 2, GV_NW, 1, true, false, PRO_LAYER, true>, dim3(max_m / 128, nseg), dim3(64 * GV_NW), 0,
                     st, P, nq, ns, 1, K, ldo);
            return launch_status();
        }
        const int wpr = MODE == 0 ? gv_waves_per_row(segs, nseg, 1, nch, tiles) : 0;
        if (wpr > 0) {
            const dim3 grid((max_m / 16 + GV_NW / wpr - 1) / (GV_NW / wpr), nseg), block(64 * GV_NW);
#define GVP(W) launch_k(k_gemv_tcq<TCQ_F32, false, W, GV_NW, 1, false, false, PRO_LAYER>, grid, block, 0, st, P, nq, ns, 1, K, ldo)
            switch (wpr) {
                case 1: GVP(1); break;
                case 2: GVP(2); break;
                case 4: GVP(4); break;
                case 8: GVP(8); break;
                default: GVP(16); break;
            }
#undef GVP
            return launch_status();
        }
        bool pairs = nw <= 8 && tiles >= 384;
        for (int i = 0; i < nseg; ++i)
            if (segs[i].rows_per_table > 0 && (segs[i].rows_per_table / 16) % 2) pairs = false;
        launch_pro_small<MODE, PRO_LAYER, TCQ_F32, 1>(max_m / 16, nseg, nw, pairs, st, P, K, ldo);
        return launch_status();
    }
    // rotate + quantize prologue, int32 sums: the streaming plan at 16 waves per tile row (the 2048 x 16384 down projection),
    // else the workgroup plan with one tile row per workgroup
    const int wpr = MODE == 0 ? gv_waves_per_row(segs, nseg, 1, nchp, tiles * parts) : 0;
    if (wpr == 16) {
        const dim3 grid(max_m / 16, nseg, parts), block(64 * GV_NW);
        if (parts == 2) launch_k(k_gemv_tcq<TCQ_I32, false, 16, GV_NW, 2, false, false, PRO_PRE>, grid, block, 0, st, P, nq, ns, 1, K, ldo);
        else launch_k(k_gemv_tcq<TCQ_I32, false, 16, GV_NW, 1, false, false, PRO_PRE>, grid, block, 0, st, P, nq, ns, 1, K, ldo);
        return launch_status();
    }
    if (parts == 2) launch_pro_small<MODE, PRO_PRE, TCQ_I32, 2>(max_m / 16, nseg, nw, false, st, P, K, ldo);
    else launch_pro_small<MODE, PRO_PRE, TCQ_I32, 1>(max_m / 16, nseg, nw, false, st, P, K, ldo);
    return launch_status();
}

extern "C" int tcq_gemm_tcq_pro(const tcq_gemm_seg* segs, int nseg, const tcq_prologue* pro, int K, int out_dtype, int ldo,
                                tcq_stream_t stream) {
    return gemm_small_pro<0>(segs, nseg, pro, K, out_dtype, ldo, stream);
}

extern "C" int tcq_gemm_w8_pro(const tcq_gemm_seg* segs, int nseg, const tcq_prologue* pro, int K, int out_dtype, int ldo,
                               tcq_stream_t stream) {
    return gemm_small_pro<1>(segs, nseg, pro, K, out_dtype, ldo, stream);
}

// ------------------------------------------------------------------------------------------ reference-shaped helpers
// The reference's small-M helpers take the activations as q4 (K/4, M) int32 words and write FP32 z (M, N)
// (deploy/tcq_kernels/kernels.py:662-673). Both run the workgroup plan of the products above with the word layout of q4;
// the fused decode reads the reference's own word layout (bits as stored, no repack) and picks table i of t8 (up to three
// concatenated (512, 2) tables) for tile rows I with (I >= nb0) + (I >= nb1) == i, as k_gemm_tcq (kernels.py:403-412).
static int small_words_check(const void* w, const int32_t* q4, int ldq, const float* s, const float* rs, const float* z, int M, int N,
                             int K) {
    if (!w || !q4 || !s || !rs || !z || M <= 0 || N <= 0 || K <= 0 || ldq < M) return TCQ_ERR_ARG;
    if (N % 16 || K % 16) return TCQ_ERR_SHAPE;
    if (M > 64) return TCQ_ERR_UNSUPPORTED;
    if ((size_t)N * K >= ((size_t)1 << 31) || (size_t)(K / 4) * ldq * 4 >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
    if ((uintptr_t)z % 16 || (uintptr_t)rs % 16 || (uintptr_t)q4 % 4) return TCQ_ERR_ALIGN;
    return TCQ_OK;
}

extern "C" int tcq_gemm_w8_q4(const int8_t* W, const int32_t* q4, int ldq, const float* s, const float* rs, float* z, int M, int N,
                              int K, tcq_stream_t stream) {
    const int e = small_words_check(W, q4, ldq, s, rs, z, M, N, K);
    if (e) return e;
    SegPack P = {};
    P.s[0] = tcq_gemm_seg{W, nullptr, rs, z, N, 0};
    const int nch = (K + 255) / 256, nw = nch < SM_MAXW ? nch : SM_MAXW;
    launch_small_qb<1, 1, QL_WORDS>(dim3(N / 16, 1), dim3(64 * nw), (hipStream_t)stream, P, (const i8*)q4, s, M, K, N, ldq, TCQ_F32);
    return launch_status();
}

extern "C" int tcq_gemm_tcq_q4(const void* bits, const int8_t* t8, const int32_t* q4, int ldq, const float* s, const float* rs,
                               float* z, int M, int N, int K, int nb0, int nb1, tcq_stream_t stream) {
    const int e = small_words_check(bits, q4, ldq, s, rs, z, M, N, K);
    if (e) return e;
    if (!t8 || nb0 < 0 || nb1 < nb0) return TCQ_ERR_ARG;
    const int tiles = N / 16, tiles_n = K / 16;
    const int bnd[4] = {0, nb0 < tiles ? nb0 : tiles, nb1 < tiles ? nb1 : tiles, tiles};
    SegPack P = {};
    int nseg = 0, max_m = 0;
    for (int i = 0; i < 3; ++i) {
        const int lo = bnd[i], hi = bnd[i + 1];
        if (hi <= lo) continue;
        P.s[nseg++] = tcq_gemm_seg{(const u16*)bits + (size_t)lo * tiles_n * 32, t8 + 1024 * i, rs + 16 * lo, z + 16 * lo, 16 * (hi - lo), 0};
        if (16 * (hi - lo) > max_m) max_m = 16 * (hi - lo);
    }
    const int nch = (K + 255) / 256, nw = nch < SM_MAXW ? nch : SM_MAXW;
    launch_small_qb<0, 1, QL_WORDS, true>(dim3(max_m / 16, nseg), dim3(64 * nw), (hipStream_t)stream, P, (const i8*)q4, s, M, K, N, ldq,
                                          TCQ_F32);
    return launch_status();
}

// ------------------------------------------------------------------------------------------------ stage-split middle
// The rest of the gated-MLP middle after a TCQ_Z_W128T product of gate | up (zt: gate's (M, 128, N / 128) block-transposed
// rows, then up's; N = 16384): block Walsh stages h = 128 .. N / 2 across the 128 blocks (h = 128 h_b), then, as tcq_mid2
// (deploy/tcq_kernels/kernels.py:263-278), * c, the signs, BF16 roundings, GELU by table and the product:
// p = bf16(gelu(bf16(g c sg)) * bf16(u c su)) (M, N) BF16 in natural order, the input of tcq_pre with the down projection's
// signs. One wave per (offset o, token t): lane l holds blocks l and l + 64 of gate and of up.
__global__ __launch_bounds__(256) void k_glu_split(const float* zt, const i8* sv, const u16* lut, u16* p, int M, int N) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int o = blockIdx.x * 4 + wave, t = blockIdx.y;
    const size_t row = ((size_t)t * 128 + o) * 128;
    const float* zg = zt + row;
    const float* zu = zt + (size_t)M * N + row;
    float v[4] = {gptr(zg)[lane], gptr(zg)[lane + 64], gptr(zu)[lane], gptr(zu)[lane + 64]};
#pragma unroll
    for (int m = 1; m <= 32; m *= 2)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float pv = lane_xor(v[e], m, lane);
            v[e] = (lane & m) ? pv - v[e] : v[e] + pv;
        }
    float a = v[0];
    v[0] = a + v[1];
    v[1] = a - v[1];
    a = v[2];
    v[2] = a + v[3];
    v[3] = a - v[3];
    const float c = (float)(1.0 / __builtin_sqrt((double)N));
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = (lane + 64 * k) * 128 + o;
        const u16 gv = gptr(lut)[f32_to_bf16(v[k] * c * (float)gptr(sv)[i])];
        const float uu = bf16_to_f32(f32_to_bf16((v[2 + k] * c) * (float)gptr(sv)[N + i]));
        gptr(p)[(size_t)t * N + i] = f32_to_bf16(bf16_to_f32(gv) * uu);
    }
}

extern "C" int tcq_glu_split(const float* zt, int N, const int8_t* sv, const uint16_t* gelu_lut, uint16_t* p, int M,
                             tcq_stream_t stream) {
    if (!zt || !sv || !gelu_lut || !p || M <= 0) return TCQ_ERR_ARG;
    if (N != 16384) return TCQ_ERR_UNSUPPORTED;
    if (M > 16) return TCQ_ERR_UNSUPPORTED;
    launch_k(k_glu_split, dim3(32, M), dim3(256), 0, (hipStream_t)stream, zt, (const i8*)sv, (const u16*)gelu_lut, (u16*)p, M, N);
    return launch_status();
}
