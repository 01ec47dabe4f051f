// Fused FP16-table decode-GEMV / small-M GEMM (M <= 16 tokens) of the TCQ 2-bit format: the packed trellis words stream
// from HBM once, are decoded per lane against an LDS codebook and feed v_mfma_f32_16x16x32_f16 with FP32 accumulation.
//
// Device layout of the words (tcq_repack): for tile row I and chunk c (16 tiles = 256 input columns) 1 KiB, in which
// dword 4 l + j of lane l = 16 g + r is the 32-bit window (word[2r] << 16) | word[2r + 1] of tile 16 c + 4 j + g. One
// buffer_load_dwordx4 per lane reads a whole chunk row, coalesced. The rest of lane r's 48-bit window, word[2r + 2], is the
// top half of lane r + 1's window (tail-biting: lane 15 -> lane 0), fetched by DPP row_ror:15.
//
// Decode of one tile row (8 weight pairs, 16 weights): windows wp_p = alignbit(hi, hn, 32 - 4p), p = 0..3, hold state p in
// their high half and state p + 4 in the low half; one v_pk_mad_u16 gives both codes x = (s + 1) s mod 2^16; table entry
// e = x >> 6 (10 bits, the sign of the first coordinate folded in as bit 9) -> one ds_read_b32 of an FP16 pair.
// Codebook in LDS: 1024 entries x C copies, entry e copy c at word e C + c, lane l reads copy l mod C. With C = 32 every
// lane of a half-wave reads its own bank, so random codes cause no bank conflicts (measured on MI355X: ~25 random lookups
// per clock per CU with 32 copies vs ~12 with one).
// MFMA mapping: A = decoded weights, lane (g, r) = row r, k-block g: A0 = pairs 0..3 of tile 16 c + 4 j + g, A1 = pairs
// 4..7; B = activations of token lr = lane % 16 at the same k, read from LDS (zero for tokens >= M and for columns >= n).
// D: lane (g, t) holds output rows 4 g .. 4 g + 3 of token t.
#include "tcq_device.h"
#include "tcq_launch.h"

namespace {

constexpr int ilog2(int v) { return v <= 1 ? 0 : 1 + ilog2(v >> 1); }

// Codebook in LDS: NE = 1024 entries with the sign of the first coordinate folded in (bit 9), or NE = 512 entries with the
// sign applied in registers; C copies, entry e copy c at word e C + c.
template <int C, int NE>
__device__ __forceinline__ void fill_table(u32* tab, const u16* tl) {
    for (int e = threadIdx.x; e < NE; e += blockDim.x) {
        const int h = e & 511;
        const u32 v = ((u32)gptr(tl)[2 * h] ^ (NE == 1024 ? (u32)(e >> 9) << 15 : 0u)) | ((u32)gptr(tl)[2 * h + 1] << 16);
        if constexpr (C % 4 == 0) {
#pragma unroll
            for (int c = 0; c < C; c += 4) *(uint4_t*)(tab + e * C + c) = uint4_t{v, v, v, v};
        } else {
#pragma unroll
            for (int c = 0; c < C; ++c) tab[e * C + c] = v;
        }
    }
}

}  // namespace

// grid (workgroups per layer, layers); workgroup x covers tile rows [x rows_per_wg, (x + 1) rows_per_wg) of its layer.
// KS = 1 (layer streams): each wave takes groups of R tile rows round-robin and walks their nch chunks. KS > 1 (a few layers,
// latency): the waves form nw / KS groups of KS, wave group g owns row group g (rows_per_wg = R nw / KS) and wave k of the
// group the chunks k, k + KS, ...; the KS partial sums meet in LDS after the loop. The words of iteration it + D are loaded
// while iteration it is decoded (D + 1 register buffers, the only vector-memory loads of the loop, so in-order vmcnt waits
// never stall on the prefetch); the first D loads are issued before the codebook fill, hiding their latency behind it.
// Dynamic LDS: h16 (M, 256 nch) FP16 with zero columns from n on, the FP32 row scales of the workgroup's rows, then for
// KS > 1 the partial sums (nw R 64 float4). Two accumulators per tile row (pairs 0..3 and 4..7) halve the MFMA dependency
// chain.
// POST (layer streams, one workgroup per layer, one table): the output rotation of tcq_post runs in the same workgroup, on the
// z rows staged in LDS (dynamic LDS then also holds M rows of lds_words(m) floats), and y = walsh(z) * sv (+ bias) is stored
// as YDT; DESC is then tcq_gemv_post_layer.
template <class DESC> __device__ __forceinline__ float* zout(const DESC& L) { return nullptr; }
template <> __device__ __forceinline__ float* zout<tcq_gemv_layer>(const tcq_gemv_layer& L) { return L.z; }

template <int C, int R, int D, int AUX, int KS, int NE = 1024, bool POST = false, class DESC = tcq_gemv_layer, int YDT = TCQ_F16>
__global__ __launch_bounds__(1024) void k_gemv_f16(const DESC* layers, const u16* h16, const float* hscale, int M,
                                                   int m, int n, int rows_per_wg) {
    __shared__ __attribute__((aligned(16))) u32 tab[NE * C];
    extern __shared__ __attribute__((aligned(16))) u32 dyn[];
    const DESC L = layers[blockIdx.y];
    const int tiles_m = m >> 4, nch = (n + 255) >> 8, np = nch << 8;
    const int I0 = blockIdx.x * rows_per_wg, I1 = min(I0 + rows_per_wg, tiles_m);
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
    const int gw = wave / KS, kw = wave % KS, ngw = nw / KS;            // row-group wave index, chunk phase
    const int lr = lane & 15, lg = lane >> 4;
    const bool tok = lr < M;
    const u32 cp4 = (u32)(lane & (C - 1)) << 2;
    constexpr int ESH = 2 + ilog2(C);                     // byte shift of an entry index
    const int ngroups = (I1 - I0 + R - 1) / R;
    const int nchw = kw < nch ? (nch - 1 - kw) / KS + 1 : 0;          // chunks of this wave per row group
    const int iters = gw < ngroups ? ((ngroups - 1 - gw) / ngw + 1) * nchw : 0;
    const rsrc_t W = make_rsrc(L.wdev, (u32)(tiles_m * nch) << 10);
    const u32 wv = (u32)lane << 4;

    float4_t acc[R][2];
    uint4_t buf[D + 1][R];
    half8_t B[4][2];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r][0] = acc[r][1] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) B[j][0] = B[j][1] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};

    // iteration counters (chunk c, group k) of the next load and the next product, advanced without divisions
    int lc = kw, lk = 0, pc = kw, pk = 0, nload = 0;
    const int lastI = tiles_m - 1;
    auto load = [&](uint4_t(&dst)[R]) {
        const int Ig = I0 + (gw + lk * ngw) * R;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int I = min(Ig + r, lastI);
            dst[r] = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(W, wv, (u32)(I * nch + min(lc, nch - 1)) << 10, AUX));
        }
        if (++nload < iters) {                   // past the end the last chunk is loaded again (never used)
            lc += KS;
            if (lc >= nch) { lc = kw; ++lk; }
        }
    };
#pragma unroll
    for (int u = 0; u < D; ++u) load(buf[u]);

    u16* hl = (u16*)dyn;
    float* sl = (float*)(dyn + (M * np >> 1));
    fill_table<C, NE>(tab, (const u16*)L.tlut + (L.rows_per_table > 0 ? (size_t)(16 * I0 / L.rows_per_table) * 1024 : 0));
    for (int i = threadIdx.x; i < (M * np) >> 3; i += blockDim.x) {      // 8 FP16 per thread-step, rows padded to np
        const int t = i / (np >> 3), k = (i - t * (np >> 3)) << 3;
        ((uint4_t*)hl)[i] = k < n ? gptr((const uint4_t*)(h16 + (size_t)t * n + k))[0] : uint4_t{0, 0, 0, 0};
    }
    const u16* rsc = (const u16*)L.row_scale;
    if (!POST)                               // POST applies the row scales to the staged z rows instead (keeps two workgroups per CU)
        for (int i = threadIdx.x; i < (I1 - I0) * 16; i += blockDim.x) sl[i] = f16_to_f32(gptr(rsc)[I0 * 16 + i]);
    __syncthreads();
    if (KS == 1 && !POST && iters == 0) return;
    const float hs = gptr(hscale)[tok ? lr : 0];
    const char* hb = (const char*)hl + (size_t)(lr * np + 16 * lg) * 2;
    float* zr = sl;                                        // POST: z rows of the layer (before the row scale), stride lds_words(m)
    const int zw = lds_words(m);

    auto epilogue = [&](int r, int Ig, const float4_t& a) {
        const int I = Ig + r;
        if (I < I1 && tok) {
            if constexpr (POST) {
#pragma unroll
                for (int e = 0; e < 4; ++e) zr[lr * zw + lds_slot(16 * I + 4 * lg + e)] = a[e] * hs;
            } else {
                const float* s = sl + (I - I0) * 16 + 4 * lg;
                float4_t o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = (a[e] * hs) * s[e];
                *gptr((float4_t*)(zout(L) + (size_t)lr * m + 16 * I + 4 * lg)) = o;
            }
        }
    };

    auto process = [&](const uint4_t(&w)[R]) {
        const int c = pc, Ig = I0 + (gw + pk * ngw) * R;
        pc += KS;
        if (pc >= nch) { pc = kw; ++pk; }
        if (tok) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                B[j][0] = *(const half8_t*)(hb + 512 * c + 128 * j);
                B[j][1] = *(const half8_t*)(hb + 512 * c + 128 * j + 16);
            }
        }
        // tile tasks q = 4 r + j, software-pipelined: the lookups of task q are issued before the products of task q - 1
        u32 va[2][8];
        auto issue = [&](int q, u32(&v)[8]) {
            const u32 hi = w[q >> 2][q & 3];
            const u32 hn = (u32)__builtin_amdgcn_mov_dpp((int)hi, 0x12F, 0xf, 0xf, false);
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const u32 x = pk_code(p == 0 ? hi : __builtin_amdgcn_alignbit(hi, hn, 32 - 4 * p));
                v[p] = *(const u32*)((const char*)tab + ((((x >> 22) & (NE - 1)) << ESH) | cp4));
                v[4 + p] = *(const u32*)((const char*)tab + ((((x >> 6) & (NE - 1)) << ESH) | cp4));
                if (NE == 512) {                       // sign of the first coordinate: bit 15 of each code
                    v[p] ^= (x >> 16) & 0x8000u;
                    v[4 + p] ^= x & 0x8000u;
                }
            }
        };
        auto consume = [&](int q, const u32(&v)[8]) {
            const uint4_t A0 = {v[0], v[1], v[2], v[3]}, A1 = {v[4], v[5], v[6], v[7]};
            acc[q >> 2][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, A0), B[q & 3][0], acc[q >> 2][0], 0, 0, 0);
            acc[q >> 2][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, A1), B[q & 3][1], acc[q >> 2][1], 0, 0, 0);
        };
        issue(0, va[0]);
#pragma unroll
        for (int q = 1; q < 4 * R; ++q) {
            issue(q, va[q & 1]);
            __builtin_amdgcn_sched_barrier(0);      // keep the products of task q - 1 after the lookups of task q
            consume(q - 1, va[(q - 1) & 1]);
        }
        consume(4 * R - 1, va[(4 * R - 1) & 1]);
        if (KS == 1 && c == nch - 1) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                epilogue(r, Ig, acc[r][0] + acc[r][1]);
                acc[r][0] = acc[r][1] = float4_t{0.f, 0.f, 0.f, 0.f};
            }
        }
    };

    for (int it0 = 0; it0 < iters; it0 += D + 1) {
#pragma unroll
        for (int u = 0; u <= D; ++u) {
            if (it0 + u < iters) {
                load(buf[(u + D) % (D + 1)]);
                process(buf[u]);
            }
        }
    }
    if constexpr (KS > 1) {                  // every wave owns at most one row group: sum the KS chunk phases in LDS
        float4_t* part = (float4_t*)(sl + rows_per_wg * 16);
#pragma unroll
        for (int r = 0; r < R; ++r) part[(wave * R + r) * 64 + lane] = acc[r][0] + acc[r][1];
        __syncthreads();
        if (kw == 0 && gw < ngroups) {
            const int Ig = I0 + gw * R;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float4_t a = part[(wave * R + r) * 64 + lane];
                for (int k = 1; k < KS; ++k) a += part[((wave + k) * R + r) * 64 + lane];
                epilogue(r, Ig, a);
            }
        }
    }
    if constexpr (POST) {                    // output rotation of every token row: walsh(z) * sv (+ bias) -> y, as tcq_post
        __syncthreads();
        for (int i = 8 * threadIdx.x; i < m; i += 8 * blockDim.x) {       // z = (acc * hs) * row scale, as the unfused epilogue
            const uint4_t rsv = *gptr((const uint4_t*)(rsc + i));
            float r8[8];
#pragma unroll
            for (int k = 0; k < 4; ++k) { r8[2 * k] = f16_to_f32((u16)(rsv[k] & 0xffffu)); r8[2 * k + 1] = f16_to_f32((u16)(rsv[k] >> 16)); }
            for (int t = 0; t < M; ++t)
#pragma unroll
                for (int k = 0; k < 8; ++k) zr[t * zw + lds_slot(i + k)] = zr[t * zw + lds_slot(i + k)] * r8[k];
        }
        __syncthreads();
        for (int t = 0; t < M; ++t) {
            float* row = zr + t * zw;
            block_walsh(row, m, [&](int i, float v) { row[lds_slot(i)] = v; });
            __syncthreads();
            for (int i = 8 * threadIdx.x; i < m; i += 8 * blockDim.x) {
                const u64 sg = *gptr((const u64*)((const i8*)L.sv + i));
                float v[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) v[k] = row[lds_slot(i + k)] * (float)(i8)(sg >> (8 * k));
                if (L.bias) {
                    const float4_t b0 = gptr((const float4_t*)(L.bias + i))[0], b1 = gptr((const float4_t*)(L.bias + i))[1];
#pragma unroll
                    for (int k = 0; k < 4; ++k) { v[k] = v[k] + b0[k]; v[4 + k] = v[4 + k] + b1[k]; }
                }
                if constexpr (YDT == TCQ_F32) {
                    float* y = (float*)L.y + (size_t)t * m + i;
                    gptr((float4_t*)y)[0] = float4_t{v[0], v[1], v[2], v[3]};
                    gptr((float4_t*)y)[1] = float4_t{v[4], v[5], v[6], v[7]};
                } else {
                    uint4_t w;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const u32 a = YDT == TCQ_BF16 ? f32_to_bf16(v[2 * k]) : f32_to_f16(v[2 * k]);
                        const u32 b = YDT == TCQ_BF16 ? f32_to_bf16(v[2 * k + 1]) : f32_to_f16(v[2 * k + 1]);
                        w[k] = a | (b << 16);
                    }
                    *gptr((uint4_t*)((u16*)L.y + (size_t)t * m + i)) = w;
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------------------------ plan
// Launch shapes (measured on MI355X).
// Stream (many tile rows, KS = 1): 16 table copies, 4 tile rows per wave, one iteration of prefetch and 512-thread
// workgroups beat 32 copies / 1024 threads and the shallower / deeper pipelines on 1024 layers of 2048 x 2048. Big layer
// counts get one workgroup per layer (the table is then filled once per layer), else the rows are split so that every
// wave of a workgroup has at least one group of rows.
// Latency (at most LAT_ROWS tile rows in the batch): one tile row per workgroup and KS = 4 / 8 / 16 waves splitting its
// chunks, so a single 2048 x 2048 layer runs as 128 workgroups of 8 waves with one 1 KiB chunk each instead of 4 workgroups
// walking 32 rows.
constexpr int GEMV_C = 16, GEMV_R = 4, GEMV_D = 1, GEMV_THREADS = 512;
constexpr int LAT_C = 8, LAT_ROWS = 2048;

struct GemvPlan {
    int rows_per_wg, wgs, threads, ks;
    size_t dyn;
};

// rpt > 0 (row-group tables of rpt rows): a workgroup of the stream plan covers one group, so it fills one table.
static GemvPlan gemv_plan(int nlayers, int M, int m, int n, int rpt) {
    const int tiles_m = m / 16, nch = (n + 255) / 256;
    const size_t hbytes = (size_t)M * nch * 256 * 2;
    GemvPlan p;
    if ((size_t)nlayers * tiles_m <= LAT_ROWS) {
        p.ks = nch >= 16 ? 16 : nch >= 8 ? 8 : 4;
        p.rows_per_wg = 1;
        p.wgs = tiles_m;
        p.threads = 64 * p.ks;
        p.dyn = hbytes + 64 + (size_t)p.ks * 1024;
        return p;
    }
    const int waves = GEMV_THREADS / 64;
    int rows;
    if (nlayers >= 256) {
        rows = tiles_m;
    } else {                                            // aim at ~512 workgroups, one group of rows per wave at least
        const int per_layer = (512 + nlayers - 1) / nlayers;
        rows = (tiles_m + per_layer - 1) / per_layer;
        if (rows < waves * GEMV_R) rows = waves * GEMV_R;
    }
    rows = (rows + GEMV_R - 1) / GEMV_R * GEMV_R;
    while (hbytes + (size_t)rows * 64 + 4096 * GEMV_C > 160 * 1024 && rows > GEMV_R) rows = (rows / 2 + GEMV_R - 1) / GEMV_R * GEMV_R;
    if (rpt > 0) rows = rpt / 16;                       // rows past a group's end are computed by its last wave but not stored
    p.ks = 1;
    p.rows_per_wg = rows;
    p.wgs = (tiles_m + rows - 1) / rows;
    p.threads = GEMV_THREADS;
    p.dyn = hbytes + (size_t)rows * 64;
    return p;
}

extern "C" int tcq_gemv_f16_groups(const tcq_gemv_layer* layers, int nlayers, const void* h16, const float* hscale, int M, int m,
                                   int n, int rows_per_table, tcq_stream_t stream) {
    if (!layers || !h16 || !hscale || nlayers <= 0 || M <= 0 || m <= 0 || n <= 0 || rows_per_table < 0) return TCQ_ERR_ARG;
    if (m % 16 || n % 16 || (rows_per_table > 0 && (rows_per_table % 16 || m % rows_per_table))) return TCQ_ERR_SHAPE;
    if (M > 16 || nlayers > 65535) return TCQ_ERR_UNSUPPORTED;
    if ((uintptr_t)h16 % 16) return TCQ_ERR_ALIGN;
    if ((size_t)(m / 16) * ((n + 255) / 256) * 1024 >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;   // one layer's words < 2 GiB
    const GemvPlan p = gemv_plan(nlayers, M, m, n, rows_per_table);
    const int C = p.ks == 1 ? GEMV_C : LAT_C;
    if (p.dyn + 4096 * C > 160 * 1024) return TCQ_ERR_UNSUPPORTED;                                // activations do not fit LDS
    constexpr int NT = 2;   // non-temporal loads: every packed word is read once
    const dim3 grid(p.wgs, nlayers), block(p.threads);
    const hipStream_t st = (hipStream_t)stream;
    const u16* h = (const u16*)h16;
    switch (p.ks) {
        case 1: launch_k(k_gemv_f16<GEMV_C, GEMV_R, GEMV_D, NT, 1>, grid, block, p.dyn, st, layers, h, hscale, M, m, n, p.rows_per_wg); break;
        case 4: launch_k(k_gemv_f16<LAT_C, 1, 1, NT, 4>, grid, block, p.dyn, st, layers, h, hscale, M, m, n, p.rows_per_wg); break;
        case 8: launch_k(k_gemv_f16<LAT_C, 1, 1, NT, 8>, grid, block, p.dyn, st, layers, h, hscale, M, m, n, p.rows_per_wg); break;
        default: launch_k(k_gemv_f16<LAT_C, 1, 1, NT, 16>, grid, block, p.dyn, st, layers, h, hscale, M, m, n, p.rows_per_wg); break;
    }
    return launch_status();
}

extern "C" int tcq_gemv_f16(const tcq_gemv_layer* layers, int nlayers, const void* h16, const float* hscale, int M, int m, int n,
                            tcq_stream_t stream) {
    return tcq_gemv_f16_groups(layers, nlayers, h16, hscale, M, m, n, 0, stream);
}

// Layer streams with the output rotation fused (POST): one workgroup per layer, single-table layers, M rows of z in LDS.
extern "C" int tcq_gemv_f16_post(const tcq_gemv_post_layer* layers, int nlayers, const void* h16, const float* hscale, int M, int m,
                                 int n, int y_dtype, tcq_stream_t stream) {
    if (!layers || !h16 || !hscale || nlayers <= 0 || M <= 0 || m <= 0 || n <= 0) return TCQ_ERR_ARG;
    if (m % 16 || n % 16 || m > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    if (M > 16 || nlayers > 65535) return TCQ_ERR_UNSUPPORTED;
    if ((uintptr_t)h16 % 16) return TCQ_ERR_ALIGN;
    if ((size_t)(m / 16) * ((n + 255) / 256) * 1024 >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
    const int tiles_m = m / 16, nch = (n + 255) / 256;
    const size_t dyn = (size_t)M * nch * 256 * 2 + (size_t)M * lds_words(m) * 4;
    if (dyn + 4096 * GEMV_C > 160 * 1024) return TCQ_ERR_UNSUPPORTED;                 // z rows / activations do not fit LDS
    constexpr int NT = 2;
    const dim3 grid(1, nlayers), block(GEMV_THREADS);
    const hipStream_t st = (hipStream_t)stream;
    const u16* h = (const u16*)h16;
#define GEMV_POST(YD) launch_k(k_gemv_f16<GEMV_C, GEMV_R, GEMV_D, NT, 1, 1024, true, tcq_gemv_post_layer, YD>, grid, block, dyn, st, \
                               layers, h, hscale, M, m, n, tiles_m)
    switch (y_dtype) {
        case TCQ_F16: GEMV_POST(TCQ_F16); break;
        case TCQ_BF16: GEMV_POST(TCQ_BF16); break;
        case TCQ_F32: GEMV_POST(TCQ_F32); break;
        default: return TCQ_ERR_DTYPE;
    }
    return launch_status();
}
