// Trellis decode kernels: load-time table snap and word repack, dense INT8 / FP16 decode, and the fused FP16-table
// decode-GEMV (small-M GEMM on MFMA) that streams the packed words from HBM.
#include "tcq_device.h"
#include "tcq_launch.h"

typedef unsigned short ushort2_t __attribute__((ext_vector_type(2)));

// x = (s + 1) s modulo 2^16 for the two 16-bit states held in w (one v_pk_mad_u16)
__device__ __forceinline__ u32 pk_code(u32 w) {
    const ushort2_t s = __builtin_bit_cast(ushort2_t, w);
    const ushort2_t x = s * s + s;
    return __builtin_bit_cast(u32, x);
}

// 48-bit window of tile row r: hi = (word[2r] << 16) | word[2r + 1], lo = word[(2r + 2) & 31]. State p (0..7) =
// bits [4p, 4p + 16) of hi:lo from the top (reference tcq_format.py:58-63; kernels.py:186-205).
__device__ __forceinline__ u32 row_state(u32 hi, u32 lo16, int p) {
    const u64 win = ((u64)hi << 16) | lo16;
    return (u32)(win >> (32 - 4 * p)) & 0xffffu;
}

// ------------------------------------------------------------------------------------------------------------------ snap
__global__ void k_snap(const u16* tlut, const u16* row_scale, int m, i8* t8, float* rs, float* gain) {
    __shared__ float red[16];
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
    for (int i = threadIdx.x; i < m; i += blockDim.x) rs[i] = f16_to_f32(row_scale[i]) / g;
    if (threadIdx.x == 0 && gain) *gain = g;
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
// One thread per (row, tile column): the 16 weights of one tile row. Sign-folded tables in LDS.
__global__ void k_decode_i8(const u16* bits, const i8* t8, i8* out, int m, int n) {
    __shared__ u16 tab[1024];
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
    if (idx >= (size_t)m * tiles) return;
    const int row = (int)(idx / tiles), J = (int)(idx % tiles), r = row & 15;
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

__global__ void k_decode_f16(const u16* bits, const u16* tlut, u16* out, int m, int n) {
    __shared__ u32 tab[1024];
    for (int e = threadIdx.x; e < 1024; e += blockDim.x) {
        const int h = e & 511;
        tab[e] = ((u32)tlut[2 * h] ^ ((u32)(e >> 9) << 15)) | ((u32)tlut[2 * h + 1] << 16);
    }
    __syncthreads();
    const int tiles = n >> 4;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)m * tiles) return;
    const int row = (int)(idx / tiles), J = (int)(idx % tiles), r = row & 15;
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

// ------------------------------------------------------------------------------------------- fused FP16-table decode-GEMV
// Work: one wave = TRW tile rows (16 output rows each) over the whole input width; a workgroup of 8 waves covers
// rows_per_wg tile rows of one layer (blockIdx.y = layer). Per chunk of 16 tiles (1 KiB of words in the device layout) each
// lane loads one dwordx4: the windows hi_r of 4 tiles (tile 16 c + 4 j + g, lane = 16 g + r). The neighbour window hi_{r+1}
// (tail-biting within the tile) comes from lane (r + 1) % 16 of the same 16-lane row by DPP row_ror:15. The 32-bit window
// starting at state p (p = 0..3) holds state p in its high half and state p + 4 in its low half, so one v_pk_mad_u16 gives
// both codes; each code indexes the sign-folded FP16-pair table in LDS. The 8 pairs of the lane's tile row are the
// A operands of two v_mfma_f32_16x16x32_f16 (k slots = the tile's columns 0..7 and 8..15, any k order works as long as the
// activations use the same one); B = activations of tokens j = lane % 16 (zero for j >= M).
template <int NCOPY, int TRW>
__global__ __launch_bounds__(512) void k_gemv_f16(const tcq_gemv_layer* layers, const u16* h16, const float* hscale, int M,
                                                  int m, int n, int rows_per_wg) {
    extern __shared__ u32 tab[];  // 1024 * NCOPY entries: entry e, copy c at e * NCOPY + c
    const tcq_gemv_layer L = layers[blockIdx.y];
    const u16* tl = (const u16*)L.tlut;
    for (int i = threadIdx.x; i < 1024 * NCOPY; i += blockDim.x) {
        const int e = i / NCOPY, h = e & 511;
        tab[i] = ((u32)tl[2 * h] ^ ((u32)(e >> 9) << 15)) | ((u32)tl[2 * h + 1] << 16);
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int lr = lane & 15, lg = lane >> 4, cp = lane & (NCOPY - 1);
    const int tiles_m = m >> 4, nch = (n + 255) >> 8;
    const int I0 = blockIdx.x * rows_per_wg, I1 = min(I0 + rows_per_wg, tiles_m);
    const uint4_t* W = (const uint4_t*)L.wdev;
    const u16* rsc = (const u16*)L.row_scale;
    for (int I = I0 + wave * TRW; I < I1; I += nwaves * TRW) {
        float4_t acc[TRW];
#pragma unroll
        for (int t = 0; t < TRW; ++t) acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
        for (int c = 0; c < nch; ++c) {
            half8_t B[4][2];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k0 = 16 * (16 * c + 4 * j + lg);
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    const int k = k0 + 8 * hf;
                    if (lr < M && k < n) B[j][hf] = *(const half8_t*)(h16 + (size_t)lr * n + k);
                    else B[j][hf] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
                }
            }
#pragma unroll
            for (int t = 0; t < TRW; ++t) {
                if (I + t >= I1) break;
                const uint4_t d = W[((size_t)(I + t) * nch + c) * 64 + lane];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const u32 hi = d[j];
                    const u32 hn = (u32)__builtin_amdgcn_mov_dpp((int)hi, 0x12F, 0xf, 0xf, false);
                    u32 a0[4], a1[4];
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        const u32 wp = p == 0 ? hi : __builtin_amdgcn_alignbit(hi, hn, 32 - 4 * p);
                        const u32 x = pk_code(wp);
                        a0[p] = tab[code_index(x >> 16) * NCOPY + cp];
                        a1[p] = tab[code_index(x & 0xffffu) * NCOPY + cp];
                    }
                    const uint4_t A0 = {a0[0], a0[1], a0[2], a0[3]}, A1 = {a1[0], a1[1], a1[2], a1[3]};
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, A0), B[j][0], acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, A1), B[j][1], acc[t], 0, 0, 0);
                }
            }
        }
        // D layout: lane = 16 g + j holds rows 4 g .. 4 g + 3 of token j
        if (lr < M) {
            const float hs = hscale[lr];
#pragma unroll
            for (int t = 0; t < TRW; ++t) {
                if (I + t >= I1) break;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int row = 16 * (I + t) + 4 * lg + e;
                    L.z[(size_t)lr * m + row] = (acc[t][e] * hs) * f16_to_f32(rsc[row]);
                }
            }
        }
    }
}

// =========================================================================================================== C ABI
extern "C" const char* tcq_version(void) { return "tcq-mi355x 0.1 (gfx950)"; }
extern "C" int tcq_max_width(void) { return TCQ_MAX_WIDTH; }

extern "C" int tcq_snap(const void* tlut, const void* row_scale, int m, int8_t* t8, float* rs, float* gain, tcq_stream_t stream) {
    if (!tlut || !row_scale || !t8 || !rs || m <= 0) return TCQ_ERR_ARG;
    launch_k(k_snap, dim3(1), dim3(256), 0, (hipStream_t)stream, (const u16*)tlut, (const u16*)row_scale, m, (i8*)t8, rs, gain);
    return launch_status();
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

extern "C" int tcq_decode_i8(const void* bits, const int8_t* t8, int8_t* out, int m, int n, tcq_stream_t stream) {
    if (!bits || !t8 || !out || m <= 0 || n <= 0) return TCQ_ERR_ARG;
    if (m % 16 || n % 16) return TCQ_ERR_SHAPE;
    if ((uintptr_t)out % 16) return TCQ_ERR_ALIGN;
    const size_t total = (size_t)m * (n / 16);
    launch_k(k_decode_i8, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, (const u16*)bits,
             (const i8*)t8, (i8*)out, m, n);
    return launch_status();
}

extern "C" int tcq_decode_f16(const void* bits, const void* tlut, void* out, int m, int n, tcq_stream_t stream) {
    if (!bits || !tlut || !out || m <= 0 || n <= 0) return TCQ_ERR_ARG;
    if (m % 16 || n % 16) return TCQ_ERR_SHAPE;
    if ((uintptr_t)out % 16) return TCQ_ERR_ALIGN;
    const size_t total = (size_t)m * (n / 16);
    launch_k(k_decode_f16, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, (const u16*)bits,
             (const u16*)tlut, (u16*)out, m, n);
    return launch_status();
}

extern "C" int tcq_gemv_f16(const tcq_gemv_layer* layers, int nlayers, const void* h16, const float* hscale, int M, int m, int n,
                            tcq_stream_t stream) {
    if (!layers || !h16 || !hscale || nlayers <= 0 || M <= 0 || m <= 0 || n <= 0) return TCQ_ERR_ARG;
    if (m % 16 || n % 16) return TCQ_ERR_SHAPE;
    if (M > 16 || nlayers > 65535) return TCQ_ERR_UNSUPPORTED;
    if ((uintptr_t)h16 % 16) return TCQ_ERR_ALIGN;
    constexpr int NCOPY = 1, TRW = 1, WAVES = 8;
    const int tiles_m = m / 16;
    // enough workgroups to fill the chip: about 1024 in total, at least one wave-row per wave
    int per_layer = (1024 + nlayers - 1) / nlayers;
    int rows_per_wg = (tiles_m + per_layer - 1) / per_layer;
    if (rows_per_wg < WAVES * TRW) rows_per_wg = WAVES * TRW < tiles_m ? WAVES * TRW : tiles_m;
    const int wgs = (tiles_m + rows_per_wg - 1) / rows_per_wg;
    launch_k(k_gemv_f16<NCOPY, TRW>, dim3(wgs, nlayers), dim3(64 * WAVES), 1024 * NCOPY * sizeof(u32), (hipStream_t)stream,
             layers, (const u16*)h16, hscale, M, m, n, rows_per_wg);
    return launch_status();
}
