// Trellis decode kernels: load-time table snap and word repack, dense INT8 / FP16 decode.
#include "tcq_device.h"
#include "tcq_launch.h"

// 48-bit window of tile row r: hi = (word[2r] << 16) | word[2r + 1], lo = word[(2r + 2) & 31]. State p (0..7) =
// bits [4p, 4p + 16) of hi:lo from the top (reference tcq_format.py:58-63; kernels.py:186-205).
__device__ __forceinline__ u32 row_state(u32 hi, u32 lo16, int p) {
    const u64 win = ((u64)hi << 16) | lo16;
    return (u32)(win >> (32 - 4 * p)) & 0xffffu;
}

// ------------------------------------------------------------------------------------------------------------------ snap
// Workgroup g snaps table g of G (row-group tables: rows [g rpt, (g + 1) rpt) read table g, rpt = m / G).
__global__ void k_snap(const u16* tlut_all, const u16* row_scale, int rpt, i8* t8_all, float* rs, float* gain) {
    __shared__ float red[16];
    const int gi = blockIdx.x;
    const u16* tlut = tlut_all + 1024 * gi;
    i8* t8 = t8_all + 1024 * gi;
    float mx = 0.f;
    for (int i = threadIdx.x; i < 1024; i += blockDim.x) mx = fmaxf(mx, fabsf(f16_to_f32(tlut[i])));
    mx = block_max(mx, red);
    // 127.0 / tensor is Tensor.__rdiv__ = reciprocal() * 127 (torch/_tensor.py), so g = float(1 / amax) * 127
    const float g = (1.0f / mx) * 127.0f;
    for (int i = threadIdx.x; i < 1024; i += blockDim.x) {
        float v = __builtin_rintf(f16_to_f32(tlut[i]) * g);
        v = fminf(fmaxf(v, -127.f), 127.f);
        t8[i] = (i8)(int)v;
    }
    for (int i = threadIdx.x; i < rpt; i += blockDim.x) rs[gi * rpt + i] = f16_to_f32(row_scale[gi * rpt + i]) / g;
    if (threadIdx.x == 0 && gain) gain[gi] = g;
}

// ---------------------------------------------------------------------------------------------------------------- repack
__global__ void k_repack(const u16* bits, u32* wdev, int m, int n, long long total) {
    const long long d = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= total) return;
    const int tiles = n >> 4, nch = (n + 255) >> 8;
    const int j = (int)(d & 3), lane = (int)((d >> 2) & 63);
    const long long blk = d >> 8;                          // (I, c) chunk index
    const int c = (int)(blk % nch), I = (int)(blk / nch);
    const int r = lane & 15, g = lane >> 4, tile = 16 * c + 4 * j + g;
    u32 v = 0;
    if (tile < tiles) {
        const u16* t = bits + ((size_t)I * tiles + tile) * 32;
        v = ((u32)t[2 * r] << 16) | (u32)t[2 * r + 1];
    }
    wdev[d] = v;
}

// --------------------------------------------------------------------------------------------------------- dense decode
// One thread per (row, tile column): the 16 weights of one tile row. Sign-folded tables in LDS. grid (blocks per row group,
// row groups): the workgroups of group g (rows [g rpt, (g + 1) rpt)) load table g.
__global__ void k_decode_i8(const u16* bits, const i8* t8_all, i8* out, int rpt, int n) {
    __shared__ u16 tab[1024];
    const i8* t8 = t8_all + 1024 * blockIdx.y;
    for (int e = threadIdx.x; e < 1024; e += blockDim.x) {
        const int h = e & 511;
        int v0 = t8[2 * h];
        const int v1 = t8[2 * h + 1];
        if (e >> 9) v0 = -v0;
        tab[e] = (u16)((v0 & 0xff) | ((v1 & 0xff) << 8));
    }
    __syncthreads();
    const int tiles = n >> 4;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)rpt * tiles) return;
    const int row = blockIdx.y * rpt + (int)(idx / tiles), J = (int)(idx % tiles), r = row & 15;
    const u16* t = bits + ((size_t)(row >> 4) * tiles + J) * 32;
    const u32 hi = ((u32)t[2 * r] << 16) | t[2 * r + 1], lo = t[(2 * r + 2) & 31];
    uint4_t w;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const u32 s0 = row_state(hi, lo, 2 * d), s1 = row_state(hi, lo, 2 * d + 1);
        w[d] = (u32)tab[code_index((s0 + 1) * s0)] | ((u32)tab[code_index((s1 + 1) * s1)] << 16);
    }
    *(uint4_t*)(out + (size_t)row * n + 16 * J) = w;
}

// Dense INT8 decode from the tcq_repack words: a wave takes one 1 KiB chunk (one tile row, 256 columns); lane (g, r)
// holds the windows of row r for tiles 16 c + 4 j + g (j = 0..3) in one dwordx4 and writes their 16 weights, so a store
// writes 64 contiguous bytes of each of the 16 rows. The lookups are those of the fused products (pk_code states, a
// sign-folded table with 16 copies, lane l reading copy l mod 16), whose 16 bytes per lane and j are the row's weights in
// column order, so the output equals k_decode_i8's byte for byte.
constexpr int DW_C = 16, DW_NW = 16;

__global__ __launch_bounds__(64 * DW_NW) void k_decode_i8_words(const u32* words, const i8* t8, i8* out, int m, int n) {
    __shared__ __attribute__((aligned(16))) u32 tab[1024 * DW_C];
    const int nch = (n + 255) >> 8, tiles = n >> 4;
    const long long chunk = (long long)blockIdx.x * DW_NW + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const bool live = chunk < (long long)(m >> 4) * nch;                 // uniform per wave
    uint4_t wa = uint4_t{0u, 0u, 0u, 0u};
    if (live) wa = gptr((const uint4_t*)(words + chunk * 256))[lane];
    for (int e = threadIdx.x; e < 1024; e += blockDim.x) {
        const int h = e & 511;
        int v0 = t8[2 * h];
        const int v1 = t8[2 * h + 1];
        if (e >> 9) v0 = -v0;
        const u32 v = (u32)(v0 & 0xff) | ((u32)(v1 & 0xff) << 8);
        const u32 vv = v | (v << 16);
#pragma unroll
        for (int c = 0; c < DW_C; c += 4) *(uint4_t*)(tab + e * DW_C + c) = uint4_t{vv, vv, vv, vv};
    }
    __syncthreads();
    if (!live) return;
    const int I = (int)(chunk / nch), c = (int)(chunk % nch);
    const u32 cp4 = (u32)(lane & (DW_C - 1)) << 2;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const u32 hi = wa[j];
        const u32 hn = (u32)__builtin_amdgcn_mov_dpp((int)hi, 0x12F, 0xf, 0xf, false);
        u32 e0[4], e1[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const u32 x = pk_code(p == 0 ? hi : __builtin_amdgcn_alignbit(hi, hn, 32 - 4 * p));
            e0[p] = *(const u16*)((const char*)tab + (((x >> 22) << 6) | cp4));            // pair p
            e1[p] = *(const u16*)((const char*)tab + ((x & 0xFFC0u) | cp4));                // pair p + 4
        }
        const int tile = 16 * c + 4 * j + g;
        if (tile < tiles)
            *gptr((uint4_t*)(out + (size_t)(16 * I + r) * n + 16 * tile)) =
                uint4_t{e0[0] | (e0[1] << 16), e0[2] | (e0[3] << 16), e1[0] | (e1[1] << 16), e1[2] | (e1[3] << 16)};
    }
}

__global__ void k_decode_f16(const u16* bits, const u16* tlut_all, u16* out, int rpt, int n) {
    __shared__ u32 tab[1024];
    const u16* tlut = tlut_all + 1024 * blockIdx.y;
    for (int e = threadIdx.x; e < 1024; e += blockDim.x) {
        const int h = e & 511;
        tab[e] = ((u32)tlut[2 * h] ^ ((u32)(e >> 9) << 15)) | ((u32)tlut[2 * h + 1] << 16);
    }
    __syncthreads();
    const int tiles = n >> 4;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)rpt * tiles) return;
    const int row = blockIdx.y * rpt + (int)(idx / tiles), J = (int)(idx % tiles), r = row & 15;
    const u16* t = bits + ((size_t)(row >> 4) * tiles + J) * 32;
    const u32 hi = ((u32)t[2 * r] << 16) | t[2 * r + 1], lo = t[(2 * r + 2) & 31];
    uint4_t w0, w1;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const u32 s = row_state(hi, lo, p);
        const u32 v = tab[code_index((s + 1) * s)];
        if (p < 4) w0[p] = v; else w1[p - 4] = v;
    }
    uint4_t* o = (uint4_t*)(out + (size_t)row * n + 16 * J);
    o[0] = w0;
    o[1] = w1;
}

// =========================================================================================================== C ABI
extern "C" const char* tcq_version(void) { return "tcq-mi355x 0.1 (gfx950)"; }
extern "C" int tcq_max_width(void) { return TCQ_MAX_WIDTH; }

// Row groups: m rows split evenly into G contiguous groups of rpt = m / G rows, each a whole number of 16-row tiles.
static bool groups_ok(int m, int G) { return G >= 1 && G <= 65535 && m % G == 0 && (m / G) % 16 == 0; }

extern "C" int tcq_snap_groups(const void* tlut, int G, const void* row_scale, int m, int8_t* t8, float* rs, float* gain,
                               tcq_stream_t stream) {
    if (!tlut || !row_scale || !t8 || !rs || m <= 0 || G <= 0) return TCQ_ERR_ARG;
    if (m % G) return TCQ_ERR_SHAPE;
    launch_k(k_snap, dim3(G), dim3(256), 0, (hipStream_t)stream, (const u16*)tlut, (const u16*)row_scale, m / G, (i8*)t8, rs, gain);
    return launch_status();
}

extern "C" int tcq_snap(const void* tlut, const void* row_scale, int m, int8_t* t8, float* rs, float* gain, tcq_stream_t stream) {
    return tcq_snap_groups(tlut, 1, row_scale, m, t8, rs, gain, stream);
}

extern "C" int64_t tcq_repack_words(int m, int n) {
    if (m <= 0 || n <= 0 || m % 16 || n % 16) return TCQ_ERR_SHAPE;
    return (int64_t)(m / 16) * ((n + 255) / 256) * 256;
}

extern "C" int tcq_repack(const void* bits, void* wdev, int m, int n, tcq_stream_t stream) {
    if (!bits || !wdev || m <= 0 || n <= 0) return TCQ_ERR_ARG;
    if (m % 16 || n % 16) return TCQ_ERR_SHAPE;
    const long long total = tcq_repack_words(m, n);
    launch_k(k_repack, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, (const u16*)bits, (u32*)wdev,
             m, n, total);
    return launch_status();
}

extern "C" int tcq_decode_i8_groups(const void* bits, const int8_t* t8, int G, int8_t* out, int m, int n, tcq_stream_t stream) {
    if (!bits || !t8 || !out || m <= 0 || n <= 0 || G <= 0) return TCQ_ERR_ARG;
    if (m % 16 || n % 16 || !groups_ok(m, G)) return TCQ_ERR_SHAPE;
    if ((uintptr_t)out % 16) return TCQ_ERR_ALIGN;
    const size_t per = (size_t)(m / G) * (n / 16);
    launch_k(k_decode_i8, dim3((unsigned)((per + 255) / 256), G), dim3(256), 0, (hipStream_t)stream, (const u16*)bits,
             (const i8*)t8, (i8*)out, m / G, n);
    return launch_status();
}

extern "C" int tcq_decode_i8_words(const void* words, const int8_t* t8, int8_t* out, int m, int n, tcq_stream_t stream) {
    if (!words || !t8 || !out || m <= 0 || n <= 0) return TCQ_ERR_ARG;
    if (m % 16 || n % 16) return TCQ_ERR_SHAPE;
    if ((uintptr_t)out % 16 || (uintptr_t)words % 16) return TCQ_ERR_ALIGN;
    const long long chunks = (long long)(m / 16) * ((n + 255) / 256);
    launch_k(k_decode_i8_words, dim3((unsigned)((chunks + DW_NW - 1) / DW_NW)), dim3(64 * DW_NW), 0, (hipStream_t)stream,
             (const u32*)words, (const i8*)t8, (i8*)out, m, n);
    return launch_status();
}

extern "C" int tcq_decode_i8(const void* bits, const int8_t* t8, int8_t* out, int m, int n, tcq_stream_t stream) {
    return tcq_decode_i8_groups(bits, t8, 1, out, m, n, stream);
}

extern "C" int tcq_decode_f16_groups(const void* bits, const void* tlut, int G, void* out, int m, int n, tcq_stream_t stream) {
    if (!bits || !tlut || !out || m <= 0 || n <= 0 || G <= 0) return TCQ_ERR_ARG;
    if (m % 16 || n % 16 || !groups_ok(m, G)) return TCQ_ERR_SHAPE;
    if ((uintptr_t)out % 16) return TCQ_ERR_ALIGN;
    const size_t per = (size_t)(m / G) * (n / 16);
    launch_k(k_decode_f16, dim3((unsigned)((per + 255) / 256), G), dim3(256), 0, (hipStream_t)stream, (const u16*)bits,
             (const u16*)tlut, (u16*)out, m / G, n);
    return launch_status();
}

extern "C" int tcq_decode_f16(const void* bits, const void* tlut, void* out, int m, int n, tcq_stream_t stream) {
    return tcq_decode_f16_groups(bits, tlut, 1, out, m, n, stream);
}
