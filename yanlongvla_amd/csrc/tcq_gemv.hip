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

// --------------------------------------------------------------------------------------------------- one-launch layer
// The whole FP16-table layer of a few tokens in one launch: the operations of tcq_pre_h16, tcq_gemv_f16 (latency plan: one
// tile row per workgroup, KS waves splitting its chunks) and tcq_post, step for step and in the same order, so y equals the
// three-launch chain bit for bit. Every workgroup issues the loads of its words, rotates the M input rows itself (a few KiB;
// no workgroup waits for another), decodes and multiplies its tile row, stores its 16 rows of z and counts itself in
// *counter with an agent-scope acquire-release add (after a workgroup barrier, so the count releases the whole workgroup's
// stores). The workgroup whose count completes the grid reads the whole z after an agent-scope acquire fence, rotates it,
// writes y and sets the counter back to zero, so a graph replays it without any reset.
// Rows of a power of two from 256 to 16 x (threads) run on registers (thread t owns elements [16 t, 16 t + 16), loaded and
// stored as 16-byte vectors when VEC); other widths run the LDS block Walsh.
struct LayerArgs {
    const void* x;
    const i8* su;
    const void* wdev;
    const u16* tlut;
    const u16* row_scale;
    const i8* sv;
    const float* bias;
    void* y;
    float* z;
    int* counter;
};

constexpr int LAYER_MAXCW = 4;      // chunks per wave: n <= 16384 with 16 waves

template <int XDT>
__device__ __forceinline__ float layer_x(const void* x, size_t i) {
    if constexpr (XDT == TCQ_F32) return gptr((const float*)x)[i];
    else if constexpr (XDT == TCQ_BF16) return bf16_to_f32(gptr((const u16*)x)[i]);
    else return f16_to_f32(gptr((const u16*)x)[i]);
}

// 16 consecutive elements of a 16-byte aligned row as FP32 (exact for every input type)
template <int XDT>
__device__ __forceinline__ void layer_x16(const void* x, size_t i, float (&v)[16]) {
    if constexpr (XDT == TCQ_F32) {
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const uint4_t a = gptr((const uint4_t*)((const float*)x + i))[h];
#pragma unroll
            for (int k = 0; k < 4; ++k) v[4 * h + k] = __uint_as_float(a[k]);
        }
    } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint4_t a = gptr((const uint4_t*)((const u16*)x + i))[h];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const u16 b = (u16)(a[k >> 1] >> (16 * (k & 1)));
                v[8 * h + k] = XDT == TCQ_BF16 ? bf16_to_f32(b) : f16_to_f32(b);
            }
        }
    }
}

__device__ __forceinline__ bool reg_row(int K) { return (K & (K - 1)) == 0 && K >= 256 && K <= 16 * (int)blockDim.x; }

template <int KS, int XDT, int YDT>
__global__ __launch_bounds__(64 * KS) void k_layer_f16(LayerArgs A, int M, int m, int n, int vec) {
    constexpr int C = LAT_C, NE = 1024, ESH = 2 + ilog2(C);
    __shared__ __attribute__((aligned(16))) u32 tab[NE * C];
    __shared__ float red[16], hsl[16];
    __shared__ int last;
    extern __shared__ __attribute__((aligned(16))) u32 dyn[];
    const int tiles_m = m >> 4, nch = (n + 255) >> 8, np = nch << 8, I = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const bool tok = lr < M;
    const u32 cp4 = (u32)(lane & (C - 1)) << 2;
    const int nchw = wave < nch ? (nch - 1 - wave) / KS + 1 : 0;
    const rsrc_t W = make_rsrc(A.wdev, (u32)(tiles_m * nch) << 10);
    // the codebook's halves first (fill_table's entries: tid + 64 KS j), so the table fill waits for them alone
    constexpr int TPT = NE / (64 * KS);
    u16 tl0[TPT], tl1[TPT];
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
        const int h = (tid + 64 * KS * j) & 511;
        tl0[j] = gptr(A.tlut)[2 * h];
        tl1[j] = gptr(A.tlut)[2 * h + 1];
    }
    // rows of 256 KS = 64 KS x 4 values (KS = 4 or 8 waves): the no-transpose engine (wave_walsh), thread t holding
    // elements [4 t, 4 t + 4); other power-of-two rows: registers (16 values per thread); the rest: the LDS block Walsh
    constexpr int WL = KS == 4 ? 10 : KS == 8 ? 11 : 0;
    const bool win = WL != 0 && vec && n == 1 << WL, wout = WL != 0 && vec && m == 1 << WL;
    const bool rin = !win && vec && reg_row(n), rout = !wout && vec && reg_row(m);
    const bool on_in = tid < (n >> 4), on_out = tid < (m >> 4);
    // token 0's input and the input signs, then the words, then the output signs / bias of the final rotation (used only
    // by the workgroup that completes the count), all issued before the table fill (the no-transpose engine keeps them in
    // xr[0], s4[0], sv4[0], b4[0])
    uint4_t xr[4], s4 = {0, 0, 0, 0}, sv4 = {0, 0, 0, 0};
    float4_t b4[4];
    if (win) {
        if constexpr (XDT == TCQ_F32) {
            xr[0] = gptr((const uint4_t*)((const float*)A.x + 4 * tid))[0];
        } else {
            const uint2_t a = gptr((const uint2_t*)((const u16*)A.x + 4 * tid))[0];
            xr[0] = uint4_t{a[0], a[1], 0, 0};
        }
        s4[0] = gptr((const u32*)(A.su + 4 * tid))[0];
    }
    if (rin && on_in) {
#pragma unroll
        for (int h = 0; h < (XDT == TCQ_F32 ? 4 : 2); ++h) xr[h] = gptr((const uint4_t*)((const char*)A.x + (size_t)16 * tid * (XDT == TCQ_F32 ? 4 : 2)))[h];
        s4 = gptr((const uint4_t*)(A.su + 16 * tid))[0];
    }
    uint4_t buf[LAYER_MAXCW];
#pragma unroll
    for (int j = 0; j < LAYER_MAXCW; ++j)
        if (j < nchw)
            buf[j] = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(W, (u32)lane << 4, (u32)(I * nch + wave + j * KS) << 10, 2));
    if (wout && A.counter) {
        sv4[0] = gptr((const u32*)(A.sv + 4 * tid))[0];
        if (A.bias) b4[0] = gptr((const float4_t*)(A.bias + 4 * tid))[0];
    }
    if (rout && on_out && A.counter) {
        sv4 = gptr((const uint4_t*)(A.sv + 16 * tid))[0];
        if (A.bias) {
#pragma unroll
            for (int h = 0; h < 4; ++h) b4[h] = gptr((const float4_t*)(A.bias + 16 * tid))[h];
        }
    }
    __builtin_amdgcn_sched_barrier(0);                            // keep these loads ahead of the table fill

    u16* hl = (u16*)dyn;                                          // h16 rows (M, np), zero from n on
    float* row = (float*)(dyn + (M * np >> 1));                   // one FP32 row (input rotation, then output rotation)
    float4_t* part = (float4_t*)(row + lds_words(max(n, m)));     // the KS waves' partial sums
#pragma unroll
    for (int j = 0; j < TPT; ++j) {                               // fill_table's entries from the loaded halves
        const int e = tid + 64 * KS * j;
        const u32 v = ((u32)tl0[j] ^ ((u32)(e >> 9) << 15)) | ((u32)tl1[j] << 16);
        if constexpr (C % 4 == 0) {
#pragma unroll
            for (int c = 0; c < C; c += 4) *(uint4_t*)(tab + e * C + c) = uint4_t{v, v, v, v};
        } else {
#pragma unroll
            for (int c = 0; c < C; ++c) tab[e * C + c] = v;
        }
    }
    // input rotation of every token row, as tcq_pre_h16: h = walsh(x * su), hscale = 2^e with amax / 2^e in [2^14, 2^15)
    float hsw = 0.f;                                              // no-transpose engine: the lane's token's hscale
    for (int t = 0; t < M; ++t) {
        float mx = 0.f;
        if (win) {
            if constexpr (WL != 0) {
                float v[4];
                uint4_t a = xr[0];
                if (t > 0) {
                    const size_t i = (size_t)t * n + 4 * tid;
                    if constexpr (XDT == TCQ_F32) {
                        a = gptr((const uint4_t*)((const float*)A.x + i))[0];
                    } else {
                        const uint2_t b = gptr((const uint2_t*)((const u16*)A.x + i))[0];
                        a = uint4_t{b[0], b[1], 0, 0};
                    }
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const u32 w = XDT == TCQ_F32 ? a[k] : a[k >> 1] >> (16 * (k & 1));
                    const float xv = XDT == TCQ_F32 ? __uint_as_float(w) : XDT == TCQ_BF16 ? bf16_to_f32((u16)w) : f16_to_f32((u16)w);
                    v[k] = xv * (float)(i8)(s4[0] >> (8 * k));
                }
                wave_walsh<2, KS>(v, row, [] { __syncthreads(); });
                const float c = (float)(1.0 / __builtin_sqrt((double)n));
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    v[k] = v[k] * c;
                    mx = fmaxf(mx, fabsf(v[k]));
                }
                // the row maximum through one barrier (red is written again only after the next token's Walsh
                // barrier, which every wave reaches after reading it here)
                mx = wave_max(mx);
                if (lane == 0) red[wave] = mx;
                __syncthreads();
                float amax = 0.f;
#pragma unroll
                for (int i = 0; i < KS; ++i) amax = fmaxf(amax, red[i]);
                int e = 0;
                if (amax > 0.f && amax < __builtin_inff()) {
                    frexpf(amax, &e);
                    e -= 15;
                }
                if (lr == t) hsw = ldexpf(1.f, e);
                // wave w holds elements [256 w, 256 w + 256), chunk w: the only h16 it multiplies (nch = KS), so
                // no barrier follows the store, only the wave's own ordering of its LDS accesses
                *(uint2_t*)(hl + t * np + 4 * tid) = uint2_t{(u32)f32_to_f16(ldexpf(v[0], -e)) | ((u32)f32_to_f16(ldexpf(v[1], -e)) << 16),
                                                       (u32)f32_to_f16(ldexpf(v[2], -e)) | ((u32)f32_to_f16(ldexpf(v[3], -e)) << 16)};
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
        } else if (rin) {
            float v[16];
            if (t > 0 && on_in) {
                layer_x16<XDT>(A.x, (size_t)t * n + 16 * tid, v);
            } else {
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    const u32 w = XDT == TCQ_F32 ? xr[k >> 2][k & 3] : xr[k >> 3][(k >> 1) & 3] >> (16 * (k & 1));
                    v[k] = XDT == TCQ_F32 ? __uint_as_float(w) : XDT == TCQ_BF16 ? bf16_to_f32((u16)w) : f16_to_f32((u16)w);
                }
            }
#pragma unroll
            for (int k = 0; k < 16; ++k) v[k] = v[k] * (float)(i8)(s4[k >> 2] >> (8 * (k & 3)));
            reg_walsh16_part(v, n, row);
            const float c = (float)(1.0 / __builtin_sqrt((double)n));
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                v[k] = v[k] * c;
                if (on_in) mx = fmaxf(mx, fabsf(v[k]));
            }
            const float amax = block_max(mx, red);
            int e = 0;
            if (amax > 0.f && amax < __builtin_inff()) {
                frexpf(amax, &e);
                e -= 15;
            }
            if (tid == 0) hsl[t] = ldexpf(1.f, e);
            if (on_in) {
                uint4_t h[2];
#pragma unroll
                for (int k = 0; k < 8; ++k) h[k >> 2][k & 3] = (u32)f32_to_f16(ldexpf(v[2 * k], -e)) | ((u32)f32_to_f16(ldexpf(v[2 * k + 1], -e)) << 16);
                *(uint4_t*)(hl + t * np + 16 * tid) = h[0];
                *(uint4_t*)(hl + t * np + 16 * tid + 8) = h[1];
            }
        } else {
            for (int i = tid; i < n; i += blockDim.x) row[lds_slot(i)] = layer_x<XDT>(A.x, (size_t)t * n + i) * (float)gptr(A.su)[i];
            __syncthreads();
            block_walsh(row, n, [&](int i, float v) { row[lds_slot(i)] = v; mx = fmaxf(mx, fabsf(v)); });
            const float amax = block_max(mx, red);
            int e = 0;
            if (amax > 0.f && amax < __builtin_inff()) {
                frexpf(amax, &e);
                e -= 15;
            }
            if (tid == 0) hsl[t] = ldexpf(1.f, e);
            for (int i = tid; i < np; i += blockDim.x) hl[t * np + i] = i < n ? f32_to_f16(ldexpf(row[lds_slot(i)], -e)) : (u16)0;
        }
        if (!win) __syncthreads();
    }
    const float hs = win ? hsw : hsl[tok ? lr : 0];
    const char* hb = (const char*)hl + (size_t)(lr * np + 16 * lg) * 2;

    float4_t acc[2] = {float4_t{0.f, 0.f, 0.f, 0.f}, float4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int j = 0; j < LAYER_MAXCW; ++j) {
        if (j >= nchw) break;
        const int c = wave + j * KS;
        half8_t B[4][2];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            B[q][0] = tok ? *(const half8_t*)(hb + 512 * c + 128 * q) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
            B[q][1] = tok ? *(const half8_t*)(hb + 512 * c + 128 * q + 16) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32 hi = buf[j][q];
            const u32 hn = (u32)__builtin_amdgcn_mov_dpp((int)hi, 0x12F, 0xf, 0xf, false);
            u32 v[8];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const u32 x = pk_code(p == 0 ? hi : __builtin_amdgcn_alignbit(hi, hn, 32 - 4 * p));
                v[p] = *(const u32*)((const char*)tab + ((((x >> 22) & (NE - 1)) << ESH) | cp4));
                v[4 + p] = *(const u32*)((const char*)tab + ((((x >> 6) & (NE - 1)) << ESH) | cp4));
            }
            const uint4_t A0 = {v[0], v[1], v[2], v[3]}, A1 = {v[4], v[5], v[6], v[7]};
            acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, A0), B[q][0], acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, A1), B[q][1], acc[1], 0, 0, 0);
        }
    }
    part[wave * 64 + lane] = acc[0] + acc[1];
    __syncthreads();
    if (wave == 0 && tok) {                                       // sum the chunk phases in wave order, then the epilogue
        float4_t a = part[lane];
        for (int k = 1; k < KS; ++k) a += part[k * 64 + lane];
        const int r0 = 16 * I + 4 * lg;
        const u64 rs4 = *gptr((const u64*)(A.row_scale + r0));
        uint4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = __float_as_uint((a[e] * hs) * f16_to_f32((u16)(rs4 >> (16 * e))));
        gptr((uint4_t*)(A.z + (size_t)lr * m + r0))[0] = o;
    }
    if (!A.counter) return;                                       // tcq_pre_gemv_f16: z is the output
    // hand-off: the barrier orders the workgroup's z stores before the count; the count is an agent-scope release (the
    // stores reach the level every XCD reads) and acquire; the workgroup that completes it reads every z row after an
    // agent-scope acquire fence
    __syncthreads();
    if (tid == 0) last = __hip_atomic_fetch_add(A.counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == (int)gridDim.x - 1;
    __syncthreads();
    if (!last) return;                                            // uniform over the workgroup
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (tid == 0) __hip_atomic_store(A.counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // output rotation of every token row, as tcq_post: y = walsh(z) * sv (+ bias)
    const rsrc_t Z = make_rsrc(A.z, (u32)(M * m) * 4);
    for (int t = 0; t < M; ++t) {
        if (wout) {
            if constexpr (WL != 0) {
                float v[4];
                const uint4_t a = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(Z, (u32)(t * m + 4 * tid) * 4, 0, 16));
#pragma unroll
                for (int k = 0; k < 4; ++k) v[k] = __uint_as_float(a[k]);
                wave_walsh<2, KS>(v, row, [] { __syncthreads(); });
                const float c = (float)(1.0 / __builtin_sqrt((double)m));
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    v[k] = (v[k] * c) * (float)(i8)(sv4[0] >> (8 * k));
                    if (A.bias) v[k] = v[k] + b4[0][k];
                }
                const size_t o = (size_t)t * m + 4 * tid;
                if constexpr (YDT == TCQ_F32) {
                    gptr((float4_t*)((float*)A.y + o))[0] = float4_t{v[0], v[1], v[2], v[3]};
                } else {
                    u32 h[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) h[k] = YDT == TCQ_BF16 ? f32_to_bf16(v[k]) : f32_to_f16(v[k]);
                    gptr((uint2_t*)((u16*)A.y + o))[0] = uint2_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
                }
            }
        } else if (rout) {
            float v[16];
            if (on_out) {
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const uint4_t a = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(Z, (u32)(t * m + 16 * tid + 4 * h) * 4, 0, 16));
#pragma unroll
                    for (int k = 0; k < 4; ++k) v[4 * h + k] = __uint_as_float(a[k]);
                }
            }
            reg_walsh16_part(v, m, row);
            if (on_out) {
                const float c = (float)(1.0 / __builtin_sqrt((double)m));
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    v[k] = (v[k] * c) * (float)(i8)(sv4[k >> 2] >> (8 * (k & 3)));
                    if (A.bias) v[k] = v[k] + b4[k >> 2][k & 3];
                }
                const size_t o = (size_t)t * m + 16 * tid;
                if constexpr (YDT == TCQ_F32) {
#pragma unroll
                    for (int h = 0; h < 4; ++h) gptr((float4_t*)((float*)A.y + o))[h] = float4_t{v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]};
                } else {
                    uint4_t w[2];
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        const u32 a = YDT == TCQ_BF16 ? f32_to_bf16(v[2 * k]) : f32_to_f16(v[2 * k]);
                        const u32 b = YDT == TCQ_BF16 ? f32_to_bf16(v[2 * k + 1]) : f32_to_f16(v[2 * k + 1]);
                        w[k >> 2][k & 3] = a | (b << 16);
                    }
                    gptr((uint4_t*)((u16*)A.y + o))[0] = w[0];
                    gptr((uint4_t*)((u16*)A.y + o))[1] = w[1];
                }
            }
        } else {
            for (int i = tid; i < m; i += blockDim.x)
                row[lds_slot(i)] = __hip_atomic_load(A.z + (size_t)t * m + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            block_walsh(row, m, [&](int i, float v) { row[lds_slot(i)] = v; });
            __syncthreads();
            for (int i = tid; i < m; i += blockDim.x) {
                float v = row[lds_slot(i)] * (float)gptr(A.sv)[i];
                if (A.bias) v = v + gptr(A.bias)[i];
                const size_t o = (size_t)t * m + i;
                if constexpr (YDT == TCQ_F32) gptr((float*)A.y)[o] = v;
                else if constexpr (YDT == TCQ_BF16) gptr((u16*)A.y)[o] = f32_to_bf16(v);
                else gptr((u16*)A.y)[o] = f32_to_f16(v);
            }
        }
        __syncthreads();
    }
}

// tcq_pre_gemv_f16 for rows of n = 256 NWP (NWP = 4 or 8: n = 1024 or 2048) with 16-byte aligned operands: one tile row
// per workgroup of 2 NWP waves. Waves 0 .. NWP - 1 rotate the token rows on the no-transpose engine (4 values per thread,
// the steps of k_layer_f16's) while waves NWP .. 2 NWP - 1 decode the tile row's NWP chunks, one each, into registers
// (steps 0 and 1 between the first token's two barriers, steps 2 and 3 beside its FP16 store); after the last row's FP16
// store the decode waves multiply, and the partial sums add in chunk order with k_layer_f16's epilogue, so z is the same
// bit for bit.
template <int XDT, int NWP>
__global__ __launch_bounds__(128 * NWP) void k_pre_gemv_wv(LayerArgs A, int M, int m) {
    constexpr int C = LAT_C, NE = 1024, ESH = 2 + ilog2(C), N = 256 * NWP, NT = 128 * NWP, TPT = NE / NT;
    __shared__ __attribute__((aligned(16))) u32 tab[NE * C];
    __shared__ __attribute__((aligned(16))) float row[N];
    __shared__ __attribute__((aligned(16))) float4_t part[NWP * 64];
    __shared__ float red[NWP], hsl[16];
    extern __shared__ __attribute__((aligned(16))) u32 dyn[];
    u16* hl = (u16*)dyn;                                          // h16 rows (M, N)
    const int tiles_m = m >> 4, I = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const bool rot = wave < NWP;                                  // uniform: a rotation wave, else the decoder of chunk c
    const int c = wave - NWP;
    const u32 cp4 = (u32)(lane & (C - 1)) << 2;
    const rsrc_t W = make_rsrc(A.wdev, (u32)(tiles_m * NWP) << 10);
    u16 tl0[TPT], tl1[TPT];                                       // the codebook's halves first
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
        const int h = (tid + NT * j) & 511;
        tl0[j] = gptr(A.tlut)[2 * h];
        tl1[j] = gptr(A.tlut)[2 * h + 1];
    }
    uint4_t xw = {0, 0, 0, 0}, wd = {0, 0, 0, 0};
    u32 sg = 0;
    if (rot) {                                                    // token 0's four values and their signs
        if constexpr (XDT == TCQ_F32) {
            xw = gptr((const uint4_t*)((const float*)A.x + 4 * tid))[0];
        } else {
            const uint2_t a = gptr((const uint2_t*)((const u16*)A.x + 4 * tid))[0];
            xw = uint4_t{a[0], a[1], 0, 0};
        }
        sg = gptr((const u32*)(A.su + 4 * tid))[0];
    } else {                                                      // the chunk's words
        wd = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(W, (u32)lane << 4, (u32)(I * NWP + c) << 10, 2));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < TPT; ++j) {                               // fill_table's entries from the loaded halves
        const int e = tid + NT * j;
        const u32 v = ((u32)tl0[j] ^ ((u32)(e >> 9) << 15)) | ((u32)tl1[j] << 16);
#pragma unroll
        for (int cc = 0; cc < C; cc += 4) *(uint4_t*)(tab + e * C + cc) = uint4_t{v, v, v, v};
    }
    uint4_t Aq[4][2];
    for (int t = 0; t < M; ++t) {
        float v[4];
        if (rot) {
            uint4_t a = xw;
            if (t > 0) {
                const size_t i = (size_t)t * N + 4 * tid;
                if constexpr (XDT == TCQ_F32) {
                    a = gptr((const uint4_t*)((const float*)A.x + i))[0];
                } else {
                    const uint2_t b = gptr((const uint2_t*)((const u16*)A.x + i))[0];
                    a = uint4_t{b[0], b[1], 0, 0};
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const u32 w = XDT == TCQ_F32 ? a[k] : a[k >> 1] >> (16 * (k & 1));
                const float xv = XDT == TCQ_F32 ? __uint_as_float(w) : XDT == TCQ_BF16 ? bf16_to_f32((u16)w) : f16_to_f32((u16)w);
                v[k] = xv * (float)(i8)(sg >> (8 * k));
            }
            wave_walsh_lanes<2>(v);
            wave_walsh_put<2, NWP>(v, row);
        }
        __syncthreads();                                          // the exchange row (at t = 0 also the table)
        if (rot) {
            wave_walsh_get<2, NWP>(v, row);
            const float cn = (float)(1.0 / __builtin_sqrt((double)N));
            float mx = 0.f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v[k] = v[k] * cn;
                mx = fmaxf(mx, fabsf(v[k]));
            }
            mx = wave_max(mx);
            if (lane == 0) red[wave] = mx;
        } else if (t == 0) {                                      // the decode waves' work, beside the rotation: steps 0, 1
#pragma unroll                                                    // here, 2 and 3 beside the FP16 store
            for (int q = 0; q < 2; ++q) {
                const u32 hi = wd[q];
                const u32 hn = (u32)__builtin_amdgcn_mov_dpp((int)hi, 0x12F, 0xf, 0xf, false);
                u32 vv[8];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const u32 x = pk_code(p == 0 ? hi : __builtin_amdgcn_alignbit(hi, hn, 32 - 4 * p));
                    vv[p] = *(const u32*)((const char*)tab + ((((x >> 22) & (NE - 1)) << ESH) | cp4));
                    vv[4 + p] = *(const u32*)((const char*)tab + ((((x >> 6) & (NE - 1)) << ESH) | cp4));
                }
                Aq[q][0] = uint4_t{vv[0], vv[1], vv[2], vv[3]};
                Aq[q][1] = uint4_t{vv[4], vv[5], vv[6], vv[7]};
            }
        }
        __syncthreads();                                          // the row maximum (red is rewritten only after the next
        if (!rot && t == 0) {                                     // token's first barrier, which follows every read here)
#pragma unroll
            for (int q = 2; q < 4; ++q) {
                const u32 hi = wd[q];
                const u32 hn = (u32)__builtin_amdgcn_mov_dpp((int)hi, 0x12F, 0xf, 0xf, false);
                u32 vv[8];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const u32 x = pk_code(p == 0 ? hi : __builtin_amdgcn_alignbit(hi, hn, 32 - 4 * p));
                    vv[p] = *(const u32*)((const char*)tab + ((((x >> 22) & (NE - 1)) << ESH) | cp4));
                    vv[4 + p] = *(const u32*)((const char*)tab + ((((x >> 6) & (NE - 1)) << ESH) | cp4));
                }
                Aq[q][0] = uint4_t{vv[0], vv[1], vv[2], vv[3]};
                Aq[q][1] = uint4_t{vv[4], vv[5], vv[6], vv[7]};
            }
        }
        if (rot) {
            float amax = 0.f;
#pragma unroll
            for (int i = 0; i < NWP; ++i) amax = fmaxf(amax, red[i]);
            int e = 0;
            if (amax > 0.f && amax < __builtin_inff()) {
                frexpf(amax, &e);
                e -= 15;
            }
            if (tid == 0) hsl[t] = ldexpf(1.f, e);
            *(uint2_t*)(hl + t * N + 4 * tid) = uint2_t{(u32)f32_to_f16(ldexpf(v[0], -e)) | ((u32)f32_to_f16(ldexpf(v[1], -e)) << 16),
                                                      (u32)f32_to_f16(ldexpf(v[2], -e)) | ((u32)f32_to_f16(ldexpf(v[3], -e)) << 16)};
        }
    }
    __syncthreads();                                              // every FP16 row and scale
    const bool tok = lr < M;
    if (!rot) {
        const char* hb = (const char*)hl + (size_t)(lr * N + 16 * lg) * 2;
        float4_t acc[2] = {float4_t{0.f, 0.f, 0.f, 0.f}, float4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const half8_t B0 = tok ? *(const half8_t*)(hb + 512 * c + 128 * q) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
            const half8_t B1 = tok ? *(const half8_t*)(hb + 512 * c + 128 * q + 16) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
            acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, Aq[q][0]), B0, acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, Aq[q][1]), B1, acc[1], 0, 0, 0);
        }
        part[c * 64 + lane] = acc[0] + acc[1];
    }
    __syncthreads();
    if (wave == 0 && tok) {                                       // the chunk sums in chunk order, then k_layer_f16's epilogue
        float4_t a = part[lane];
        for (int k = 1; k < NWP; ++k) a += part[k * 64 + lane];
        const float hs = hsl[lr];
        const int r0 = 16 * I + 4 * lg;
        const u64 rs4 = *gptr((const u64*)(A.row_scale + r0));
        uint4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = __float_as_uint((a[e] * hs) * f16_to_f32((u16)(rs4 >> (16 * e))));
        gptr((uint4_t*)(A.z + (size_t)lr * m + r0))[0] = o;
    }
}

// counter NULL: the launch stops after z (tcq_pre_gemv_f16; sv, bias and y unused)
static int layer_f16(const void* x, int x_dtype, const int8_t* su, const void* wdev, const void* tlut, const void* row_scale,
                     const int8_t* sv, const float* bias, void* y, int y_dtype, int M, int m, int n, float* z, int* counter,
                     tcq_stream_t stream) {
    if (m % 16 || n % 16 || m > TCQ_MAX_WIDTH || n > TCQ_MAX_WIDTH) return TCQ_ERR_SHAPE;
    if (M > 16 || m / 16 > 65535) return TCQ_ERR_UNSUPPORTED;
    if ((size_t)(m / 16) * ((n + 255) / 256) * 1024 >= ((size_t)1 << 31)) return TCQ_ERR_SHAPE;
    const int nch = (n + 255) / 256, ks = nch >= 16 ? 16 : nch >= 8 ? 8 : 4;   // the latency plan's split of a tile row
    if (nch > ks * LAYER_MAXCW) return TCQ_ERR_UNSUPPORTED;
    if ((uintptr_t)z % 16 || (uintptr_t)row_scale % 8) return TCQ_ERR_ALIGN;
    const size_t dyn = (size_t)M * nch * 256 * 2 + (size_t)lds_words(n > m ? n : m) * 4 + (size_t)ks * 64 * 16;
    if (dyn + 4096 * LAT_C + 256 > 160 * 1024) return TCQ_ERR_UNSUPPORTED;
    const LayerArgs a{x, su, wdev, (const u16*)tlut, (const u16*)row_scale, sv, bias, y, z, counter};
    const int xs = x_dtype == TCQ_F32 ? 4 : 2, ys = y_dtype == TCQ_F32 ? 4 : 2;
    const int vec = (uintptr_t)x % 16 == 0 && (uintptr_t)su % 16 == 0 && (uintptr_t)sv % 16 == 0 && (uintptr_t)y % 16 == 0 &&
                    (uintptr_t)z % 16 == 0 && (uintptr_t)bias % 16 == 0 && (size_t)n * xs % 16 == 0 && (size_t)m * ys % 16 == 0;
    const dim3 grid(m / 16), block(64 * ks);
    const hipStream_t st = (hipStream_t)stream;
    if (!counter && vec && (n == 1024 || n == 2048)) {            // rotation and decode on separate waves
        const size_t hb = (size_t)M * n * 2;
#define PGW(XD)                                                                                                            \
    if (n == 1024) launch_k(k_pre_gemv_wv<XD, 4>, grid, dim3(512), hb, st, a, M, m);                                       \
    else launch_k(k_pre_gemv_wv<XD, 8>, grid, dim3(1024), hb, st, a, M, m)
        switch (x_dtype) {
            case TCQ_F16: PGW(TCQ_F16); break;
            case TCQ_BF16: PGW(TCQ_BF16); break;
            case TCQ_F32: PGW(TCQ_F32); break;
            default: return TCQ_ERR_DTYPE;
        }
#undef PGW
        return launch_status();
    }
#define LAYER_K(KS, XD, YD) launch_k(k_layer_f16<KS, XD, YD>, grid, block, dyn, st, a, M, m, n, vec)
#define LAYER_Y(KS, XD)                                      \
    switch (y_dtype) {                                       \
        case TCQ_F16: LAYER_K(KS, XD, TCQ_F16); break;       \
        case TCQ_BF16: LAYER_K(KS, XD, TCQ_BF16); break;     \
        case TCQ_F32: LAYER_K(KS, XD, TCQ_F32); break;       \
        default: return TCQ_ERR_DTYPE;                       \
    }
#define LAYER_X(KS)                                          \
    switch (x_dtype) {                                       \
        case TCQ_F16: LAYER_Y(KS, TCQ_F16); break;           \
        case TCQ_BF16: LAYER_Y(KS, TCQ_BF16); break;         \
        case TCQ_F32: LAYER_Y(KS, TCQ_F32); break;           \
        default: return TCQ_ERR_DTYPE;                       \
    }
    switch (ks) {
        case 4: LAYER_X(4); break;
        case 8: LAYER_X(8); break;
        default: LAYER_X(16); break;
    }
#undef LAYER_X
#undef LAYER_Y
#undef LAYER_K
    return launch_status();
}

extern "C" int tcq_layer_f16(const void* x, int x_dtype, const int8_t* su, const void* wdev, const void* tlut, const void* row_scale,
                             const int8_t* sv, const float* bias, void* y, int y_dtype, int M, int m, int n, float* z, int* counter,
                             tcq_stream_t stream) {
    if (!x || !su || !wdev || !tlut || !row_scale || !sv || !y || !z || !counter || M <= 0 || m <= 0 || n <= 0) return TCQ_ERR_ARG;
    return layer_f16(x, x_dtype, su, wdev, tlut, row_scale, sv, bias, y, y_dtype, M, m, n, z, counter, stream);
}

extern "C" int tcq_pre_gemv_f16(const void* x, int x_dtype, const int8_t* su, const void* wdev, const void* tlut, const void* row_scale,
                                int M, int m, int n, float* z, tcq_stream_t stream) {
    if (!x || !su || !wdev || !tlut || !row_scale || !z || M <= 0 || m <= 0 || n <= 0) return TCQ_ERR_ARG;
    return layer_f16(x, x_dtype, su, wdev, tlut, row_scale, nullptr, nullptr, nullptr, TCQ_F16, M, m, n, z, nullptr, stream);
}
