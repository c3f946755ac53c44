// GGUF block-quantized weights (ggml block formats) on the reference's
// launcher signatures:
//   gg_gemv_kernel      gemm_q (cuda/kernels.cuh:63-66): y[n,out] = x[n,in] . W^T (+ bias),
//                       W [out, in] rows of GGUF blocks at qW + o * row_bytes.
//   gg_moe_kernel       moe_expert_ffn_q (cuda/kernels.cuh:117-123, cuda/qgemm.cu:1505-1639):
//                       gate/up rows [E, moe_inter, hidden], down [E, hidden, moe_inter],
//                       row o of expert e at base + (e * out + o) * row_bytes.
//                       Phase 1: h_act[r, f] = silu(gate_e[f] . x_t) * (up_e[f] . x_t) for
//                       every routed row r = t * topk + s; phase 2: dpart[r, o] =
//                       down_e[o] . h_act[r]; then out[t] = sum_s w[t, s] * dpart[t*topk+s]
//                       in slot order (the reference's fixed-order reduce,
//                       cuda/qgemm.cu:943-955).
// Element decode restates src/gguf_quant.cpp:98-262 per 8 consecutive elements
// with the same float operations in the same order, so the dequantized
// weights equal the reference's bit for bit; products and sums are fp32.
//
// Work: a workgroup (4 waves) owns 16 output rows (4 per wave) and a tile of
// up to 8 input rows. With the caller's `dispatch` scratch the routed rows are
// first grouped by expert (counting pass, one workgroup), so a tile holds up
// to 8 rows of one expert and each weight row is read once per tile; without
// it every routed row is a tile of its own (the reference's token-major path).
// K is walked in chunks: the tile's input rows of a chunk are staged in LDS
// (shared by the waves); each lane takes 8 consecutive K of the wave's weight
// rows and accumulates 8-element dot products; lane partials are added by a
// fixed xor butterfly. For the block types with dword-aligned rows the weight
// bytes are streamed one chunk ahead (gg_dots_stream); otherwise each lane
// reads its blocks' bytes directly (gg_dots / gg_dots_i8).
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace glmmoe {

// ggml's IQ3_XXS codebook (256 entries of 4 magnitudes, one byte each) and
// IQ4_NL values: format data, identical to the reference's tables
// (src/gguf_quant.cpp:53-90).
__constant__ uint32_t c_iq3xxs_grid[256] = {
    0x04040404u, 0x04040414u, 0x04040424u, 0x04040c0cu, 0x04040c1cu, 0x04040c3eu, 0x04041404u, 0x04041414u,
    0x04041c0cu, 0x04042414u, 0x04043e1cu, 0x04043e2cu, 0x040c040cu, 0x040c041cu, 0x040c0c04u, 0x040c0c14u,
    0x040c140cu, 0x040c142cu, 0x040c1c04u, 0x040c1c14u, 0x040c240cu, 0x040c2c24u, 0x040c3e04u, 0x04140404u,
    0x04140414u, 0x04140424u, 0x04140c0cu, 0x04141404u, 0x04141414u, 0x04141c0cu, 0x04141c1cu, 0x04141c3eu,
    0x04142c0cu, 0x04142c3eu, 0x04143e2cu, 0x041c040cu, 0x041c043eu, 0x041c0c04u, 0x041c0c14u, 0x041c142cu,
    0x041c3e04u, 0x04240c1cu, 0x04241c3eu, 0x04242424u, 0x04242c3eu, 0x04243e1cu, 0x04243e2cu, 0x042c040cu,
    0x042c043eu, 0x042c1c14u, 0x042c2c14u, 0x04341c2cu, 0x04343424u, 0x043e0c04u, 0x043e0c24u, 0x043e0c34u,
    0x043e241cu, 0x043e340cu, 0x0c04040cu, 0x0c04041cu, 0x0c040c04u, 0x0c040c14u, 0x0c04140cu, 0x0c04141cu,
    0x0c041c04u, 0x0c041c14u, 0x0c041c24u, 0x0c04243eu, 0x0c042c04u, 0x0c0c0404u, 0x0c0c0414u, 0x0c0c0c0cu,
    0x0c0c1404u, 0x0c0c1414u, 0x0c14040cu, 0x0c14041cu, 0x0c140c04u, 0x0c140c14u, 0x0c14140cu, 0x0c141c04u,
    0x0c143e14u, 0x0c1c0404u, 0x0c1c0414u, 0x0c1c1404u, 0x0c1c1c0cu, 0x0c1c2434u, 0x0c1c3434u, 0x0c24040cu,
    0x0c24042cu, 0x0c242c04u, 0x0c2c1404u, 0x0c2c1424u, 0x0c2c2434u, 0x0c2c3e0cu, 0x0c34042cu, 0x0c3e1414u,
    0x0c3e2404u, 0x14040404u, 0x14040414u, 0x14040c0cu, 0x14040c1cu, 0x14041404u, 0x14041414u, 0x14041434u,
    0x14041c0cu, 0x14042414u, 0x140c040cu, 0x140c041cu, 0x140c042cu, 0x140c0c04u, 0x140c0c14u, 0x140c140cu,
    0x140c1c04u, 0x140c341cu, 0x140c343eu, 0x140c3e04u, 0x14140404u, 0x14140414u, 0x14140c0cu, 0x14140c3eu,
    0x14141404u, 0x14141414u, 0x14141c3eu, 0x14142404u, 0x14142c2cu, 0x141c040cu, 0x141c0c04u, 0x141c0c24u,
    0x141c3e04u, 0x141c3e24u, 0x14241c2cu, 0x14242c1cu, 0x142c041cu, 0x142c143eu, 0x142c240cu, 0x142c3e24u,
    0x143e040cu, 0x143e041cu, 0x143e0c34u, 0x143e242cu, 0x1c04040cu, 0x1c040c04u, 0x1c040c14u, 0x1c04140cu,
    0x1c04141cu, 0x1c042c04u, 0x1c04342cu, 0x1c043e14u, 0x1c0c0404u, 0x1c0c0414u, 0x1c0c1404u, 0x1c0c1c0cu,
    0x1c0c2424u, 0x1c0c2434u, 0x1c14040cu, 0x1c14041cu, 0x1c140c04u, 0x1c14142cu, 0x1c142c14u, 0x1c143e14u,
    0x1c1c0c0cu, 0x1c1c1c1cu, 0x1c241c04u, 0x1c24243eu, 0x1c243e14u, 0x1c2c0404u, 0x1c2c0434u, 0x1c2c1414u,
    0x1c2c2c2cu, 0x1c340c24u, 0x1c341c34u, 0x1c34341cu, 0x1c3e1c1cu, 0x1c3e3404u, 0x24040424u, 0x24040c3eu,
    0x24041c2cu, 0x24041c3eu, 0x24042c1cu, 0x24042c3eu, 0x240c3e24u, 0x24141404u, 0x24141c3eu, 0x24142404u,
    0x24143404u, 0x24143434u, 0x241c043eu, 0x241c242cu, 0x24240424u, 0x24242c0cu, 0x24243424u, 0x242c142cu,
    0x242c241cu, 0x242c3e04u, 0x243e042cu, 0x243e0c04u, 0x243e0c14u, 0x243e1c04u, 0x2c040c14u, 0x2c04240cu,
    0x2c043e04u, 0x2c0c0404u, 0x2c0c0434u, 0x2c0c1434u, 0x2c0c2c2cu, 0x2c140c24u, 0x2c141c14u, 0x2c143e14u,
    0x2c1c0414u, 0x2c1c2c1cu, 0x2c240c04u, 0x2c24141cu, 0x2c24143eu, 0x2c243e14u, 0x2c2c0414u, 0x2c2c1c0cu,
    0x2c342c04u, 0x2c3e1424u, 0x2c3e2414u, 0x34041424u, 0x34042424u, 0x34042434u, 0x34043424u, 0x340c140cu,
    0x340c340cu, 0x34140c3eu, 0x34143424u, 0x341c1c04u, 0x341c1c34u, 0x34242424u, 0x342c042cu, 0x342c2c14u,
    0x34341c1cu, 0x343e041cu, 0x343e140cu, 0x3e04041cu, 0x3e04042cu, 0x3e04043eu, 0x3e040c04u, 0x3e041c14u,
    0x3e042c14u, 0x3e0c1434u, 0x3e0c2404u, 0x3e140c14u, 0x3e14242cu, 0x3e142c14u, 0x3e1c0404u, 0x3e1c0c2cu,
    0x3e1c1c1cu, 0x3e1c3404u, 0x3e24140cu, 0x3e24240cu, 0x3e2c0404u, 0x3e2c0414u, 0x3e2c1424u, 0x3e341c04u,
};
constexpr int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                               1,    13,   25,  38,  53,  69,  89,  113};
constexpr uint32_t iq4nl_word(int i) {
    return (uint32_t)(uint8_t)kIq4nl[4 * i] | ((uint32_t)(uint8_t)kIq4nl[4 * i + 1] << 8) |
           ((uint32_t)(uint8_t)kIq4nl[4 * i + 2] << 16) | ((uint32_t)(uint8_t)kIq4nl[4 * i + 3] << 24);
}

// IQ4_NL values of four 4-bit codes (one per byte of `codes`), packed as int8:
// two byte selects (v_perm_b32) from the table held in four constant words.
__device__ __forceinline__ uint32_t gg_iq4nl4(uint32_t codes) {
    const uint32_t sel = codes & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(iq4nl_word(1), iq4nl_word(0), sel);
    const uint32_t hi = __builtin_amdgcn_perm(iq4nl_word(3), iq4nl_word(2), sel);
    const uint32_t m = ((codes >> 3) & 0x01010101u) * 0xffu;
    return (lo & ~m) | (hi & m);
}

__device__ __forceinline__ float gg_f16(const uint8_t* p) {
    const uint16_t h = (uint16_t)(p[0] | (p[1] << 8));
    return (float)__builtin_bit_cast(_Float16, h);
}

int gguf_block_elems(uint32_t t) {
    switch (t) {
        case 0: case 1: return 1;
        case 8: return 32;
        case 11: case 12: case 13: case 14: case 18: case 23: return 256;
        default: return 0;
    }
}

int gguf_block_bytes(uint32_t t) {
    switch (t) {
        case 0: return 4;
        case 1: return 2;
        case 8: return 34;
        case 11: return 110;
        case 12: return 144;
        case 13: return 176;
        case 14: return 210;
        case 18: return 98;
        case 23: return 136;
        default: return 0;
    }
}

__device__ __forceinline__ uint32_t gg_ld32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// The codes of IQ4_XS elements k .. k + 7 of a block (k % 8 == 0), one per byte.
__device__ __forceinline__ void gg_iq4xs_codes(const uint8_t* b, int ib, int c, uint32_t& c0,
                                               uint32_t& c1) {
    const uint8_t* q = b + 8 + 16 * ib + (c % 16);
    const int sh = 4 * (c / 16);
    c0 = (gg_ld32(q) >> sh) & 0x0f0f0f0fu;
    c1 = (gg_ld32(q + 4) >> sh) & 0x0f0f0f0fu;
}

// Elements k .. k + 7 (k % 8 == 0) of a row of GGUF type t; grid: the IQ3_XXS
// codebook (constant memory or an LDS copy).
__device__ __forceinline__ void gg_dec8_any(uint32_t t, const uint8_t* __restrict__ row, int k,
                                            const uint32_t* __restrict__ grid, float (&y)[8]) {
    switch (t) {
        case 0: {
            const float4* p = reinterpret_cast<const float4*>(row + 4 * (size_t)k);
            const float4 a = p[0], b = p[1];
            y[0] = a.x; y[1] = a.y; y[2] = a.z; y[3] = a.w;
            y[4] = b.x; y[5] = b.y; y[6] = b.z; y[7] = b.w;
            return;
        }
        case 1: {
#pragma unroll
            for (int j = 0; j < 8; ++j) y[j] = gg_f16(row + 2 * ((size_t)k + j));
            return;
        }
        case 8: {   // d, 32 x int8
            const uint8_t* b = row + (size_t)(k / 32) * 34;
            const int p = k % 32;
            const float d = gg_f16(b);
#pragma unroll
            for (int j = 0; j < 8; ++j) y[j] = d * (float)(int8_t)b[2 + p + j];
            return;
        }
        case 11: {  // hmask[32] q[64] scales[12] d
            const uint8_t* b = row + (size_t)(k / 256) * 110;
            const int p = k % 256, half = p / 128, r = p % 128, j = r / 32, sub = (r % 32) / 16;
            const int l0 = r % 16, i = 8 * half + 2 * j + sub;
            const int lo = (b[96 + i % 8] >> (4 * (i / 8))) & 15;
            const int hi = (b[104 + i % 4] >> (2 * (i / 4))) & 3;
            const int sc = (int)(int8_t)(uint8_t)(lo | (hi << 4));
            const float dl = gg_f16(b + 108) * (float)(sc - 32);
            const int hm = 1 << (4 * half + j);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int idx = 16 * sub + l0 + e;
                const int v = (b[32 + 32 * half + idx] >> (2 * j)) & 3;
                y[e] = dl * (float)(v - ((b[idx] & hm) ? 0 : 4));
            }
            return;
        }
        case 12:
        case 13: {  // d dmin scales[12] (qh[32]) q[128]
            const int bb = t == 12 ? 144 : 176;
            const uint8_t* b = row + (size_t)(k / 256) * bb;
            const int p = k % 256, c64 = p / 64, c = p % 64, l0 = c % 32, hi = c / 32;
            const int js = 2 * c64 + hi;
            const uint8_t* s = b + 4;
            int sc, mn;
            if (js < 4) {
                sc = s[js] & 63;
                mn = s[js + 4] & 63;
            } else {
                sc = (s[js + 4] & 15) | ((s[js - 4] >> 6) << 4);
                mn = (s[js + 4] >> 4) | ((s[js] >> 6) << 4);
            }
            const float d1 = gg_f16(b) * (float)sc, m1 = gg_f16(b + 2) * (float)mn;
            const uint8_t* q = b + (t == 12 ? 16 : 48);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                int v = (q[32 * c64 + l0 + e] >> (4 * hi)) & 15;
                if (t == 13) v += (b[16 + l0 + e] & (1 << js)) ? 16 : 0;
                y[e] = d1 * (float)v - m1;
            }
            return;
        }
        case 14: {  // ql[128] qh[64] scales[16] d
            const uint8_t* b = row + (size_t)(k / 256) * 210;
            const int p = k % 256, nn = p / 128, r = p % 128, quarter = r / 32, l0 = r % 32;
            const uint8_t* ql = b + 64 * nn + 32 * (quarter & 1);
            const uint8_t* qh = b + 128 + 32 * nn;
            const float dsc = gg_f16(b + 208) * (float)(int8_t)b[192 + 8 * nn + l0 / 16 + 2 * quarter];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int lo = (ql[l0 + e] >> (4 * (quarter >> 1))) & 15;
                const int q6 = (int)(int8_t)(uint8_t)(lo | (((qh[l0 + e] >> (2 * quarter)) & 3) << 4)) - 32;
                y[e] = dsc * (float)q6;
            }
            return;
        }
        case 18: {  // d qs[64] signs+scales[32]
            const uint8_t* b = row + (size_t)(k / 256) * 98;
            const int p = k % 256, ib = p / 32, l = (p % 32) / 8;
            const uint8_t* w = b + 66 + 4 * ib;
            const uint32_t aux = (uint32_t)w[0] | ((uint32_t)w[1] << 8) | ((uint32_t)w[2] << 16) |
                                 ((uint32_t)w[3] << 24);
            const float db = gg_f16(b) * (0.5f + (float)(aux >> 28)) * 0.5f;
            const uint32_t i7 = (aux >> (7 * l)) & 127u;
            const uint32_t signs = i7 | ((uint32_t)(__builtin_popcount(i7) & 1) << 7);
            const uint32_t g0 = grid[b[2 + 8 * ib + 2 * l]];
            const uint32_t g1 = grid[b[2 + 8 * ib + 2 * l + 1]];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float mag = (float)(((e < 4 ? g0 : g1) >> (8 * (e & 3))) & 255u);
                y[e] = db * mag * ((signs & (1u << e)) ? -1.0f : 1.0f);
            }
            return;
        }
        case 23: {  // d scales_h scales_l[4] qs[128]
            const uint8_t* b = row + (size_t)(k / 256) * 136;
            const int p = k % 256, ib = p / 32, c = p % 32;
            const int sh = b[2] | (b[3] << 8);
            const int lo = (b[4 + ib / 2] >> (4 * (ib & 1))) & 15;
            const int hi = (sh >> (2 * ib)) & 3;
            const float dl = gg_f16(b) * (float)((int)(int8_t)(uint8_t)(lo | (hi << 4)) - 32);
            uint32_t c0, c1;
            gg_iq4xs_codes(b, ib, c, c0, c1);
            const uint32_t v0 = gg_iq4nl4(c0), v1 = gg_iq4nl4(c1);
#pragma unroll
            for (int e = 0; e < 8; ++e)
                y[e] = dl * (float)(int8_t)(((e < 4 ? v0 : v1) >> (8 * (e & 3))) & 255u);
            return;
        }
        default:
#pragma unroll
            for (int e = 0; e < 8; ++e) y[e] = 0.0f;
    }
}

// The type as a compile-time constant (one decode body per kernel
// instantiation); kGgAny decodes by a runtime switch on t.
constexpr uint32_t kGgAny = 0xffffffffu;
template <uint32_t T>
__device__ __forceinline__ void gg_dec8(uint32_t t, const uint8_t* __restrict__ row, int k,
                                        const uint32_t* __restrict__ grid, float (&y)[8]) {
    gg_dec8_any(T == kGgAny ? t : T, row, k, grid, y);
}

constexpr int kGgWaves = 4;                // waves per workgroup
constexpr int kGgThreads = 64 * kGgWaves;
constexpr int kGgRows = 4 * kGgWaves;      // weight rows per workgroup (4 per wave)
constexpr int kGgKC = 512;    // K per staged chunk
// Input rows per tile (TT): 8 for prefill-sized groups, fewer when an expert
// holds a row or a few (decode), so no FMAs go to empty rows.

__device__ __forceinline__ float gg_wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

__device__ __forceinline__ float gg_silu(float v) { return v / (1.0f + expf(-v)); }

// The input rows of a tile (up to TT, indices into src) and its expert.
template <int TT>
struct GgTile {
    int e, nr;
    int row[TT];    // output row index (routed row r, or the token for gemm_q)
    int src[TT];    // input row index into src
};

// Stages rows srcs[0..nr) x [k0, k0 + kc) of a [*, K] fp32 matrix into xs
// (srcs: the tile's input rows, in LDS so that they index dynamically).
template <int TT>
__device__ __forceinline__ void gg_stage(float (*xs)[kGgKC], const float* __restrict__ src, int K,
                                         const int* srcs, int nr, int k0, int kc) {
    for (int i = threadIdx.x; i < TT * (kGgKC / 4); i += blockDim.x) {
        const int t = i / (kGgKC / 4), c4 = i % (kGgKC / 4);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t < nr && 4 * c4 < kc)
            v = *reinterpret_cast<const float4*>(src + (size_t)srcs[t] * K + k0 + 4 * c4);
        *reinterpret_cast<float4*>(&xs[t][4 * c4]) = v;
    }
}

// Dot products of NM weight matrices' rows o0 .. o0 + 3 with the tile's input
// rows over K: acc[m][r][t].
template <uint32_t T, int NM, int TT>
__device__ __forceinline__ void gg_dots(float (*xs)[kGgKC], int* srcs, const float* __restrict__ src,
                                        int K, const GgTile<TT>& tl, const uint32_t (&type)[NM],
                                        const uint8_t* const (&wrow)[NM][4],
                                        float (&acc)[NM][4][TT]) {
    const int lane = threadIdx.x & 63;
    __syncthreads();   // srcs and xs of a previous tile are consumed
    if (threadIdx.x == 0) {
#pragma unroll
        for (int t = 0; t < TT; ++t) srcs[t] = tl.src[t];
    }
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int t = 0; t < TT; ++t) acc[m][r][t] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += kGgKC) {
        const int kc = min(kGgKC, K - k0);
        __syncthreads();
        gg_stage<TT>(xs, src, K, srcs, tl.nr, k0, kc);
        __syncthreads();
        const int kk = lane * 8;
        if (kk >= kc) continue;
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float w[8];
                gg_dec8<T>(type[m], wrow[m][r], k0 + kk, c_iq3xxs_grid, w);
#pragma unroll
                for (int j = 0; j < 8; ++j)
#pragma unroll
                    for (int t = 0; t < TT; ++t)
                        acc[m][r][t] = __builtin_fmaf(w[j], xs[t][kk + j], acc[m][r][t]);
            }
    }
}

// ---- int8 activations (gemm_q_i8 / moe_expert_ffn_q_i8, cuda/qgemm.cu:104-303,
// 556-587). Weights k .. k + 7 as integers with one affine pair,
// weight[j] = ds * wq[j] - dm (dm != 0 for Q4_K / Q5_K only), packed four
// per int32 for v_dot4c_i32_i8. The same bits give exactly the decode above.
__device__ __forceinline__ int gg_pk4(int a, int b, int c, int d) {
    return (a & 255) | ((b & 255) << 8) | ((c & 255) << 16) | (int)((unsigned)d << 24);
}


// A2: every 2- and 4-byte field is read as 16-bit halves (the caller's rows
// are 2-byte aligned, as in the LDS copies; block sizes are even); otherwise
// byte by byte.
template <bool A2>
__device__ __forceinline__ uint32_t gg_rd32(const uint8_t* p) {
    if constexpr (A2) {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
        return (uint32_t)h[0] | ((uint32_t)h[1] << 16);
    } else {
        return gg_ld32(p);
    }
}
template <bool A2>
__device__ __forceinline__ float gg_rdf16(const uint8_t* p) {
    if constexpr (A2)
        return (float)__builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t*>(p));
    else
        return gg_f16(p);
}

// Byte i of the result is 0xff where bit i of s (i < 4) is set.
__device__ __forceinline__ uint32_t gg_bytemask4(uint32_t s) {
    return (((s & 15u) * 0x00204081u) & 0x01010101u) * 0xffu;
}

// sgn (used with A2): the IQ3_XXS sign byte masks of the 128 7-bit patterns,
// two words per pattern (the LDS table of gg_dots_stream).
template <bool A2>
__device__ __forceinline__ void gg_dec8i_any(uint32_t t, const uint8_t* __restrict__ row, int k,
                                             const uint32_t* __restrict__ grid,
                                             const uint32_t* __restrict__ sgn, int& w0, int& w1,
                                             float& ds, float& dm) {
    dm = 0.0f;
    switch (t) {
        case 8: {
            const uint8_t* b = row + (size_t)(k / 32) * 34;
            ds = gg_rdf16<A2>(b);
            w0 = (int)gg_rd32<A2>(b + 2 + k % 32);
            w1 = (int)gg_rd32<A2>(b + 6 + k % 32);
            return;
        }
        case 11: {
            const uint8_t* b = row + (size_t)(k / 256) * 110;
            const int p = k % 256, half = p / 128, r = p % 128, j = r / 32, sub = (r % 32) / 16;
            const int l0 = r % 16, i = 8 * half + 2 * j + sub;
            const int lo = (b[96 + i % 8] >> (4 * (i / 8))) & 15;
            const int hi = (b[104 + i % 4] >> (2 * (i / 4))) & 3;
            ds = gg_rdf16<A2>(b + 108) * (float)((int)(int8_t)(uint8_t)(lo | (hi << 4)) - 32);
            const int idx = 16 * sub + l0, hb = 4 * half + j;
            // q - (hmask bit ? 0 : 4) per byte, q in 0..3: biased by 0x80 so no
            // byte borrows from its neighbour
            const uint32_t q0 = (gg_rd32<A2>(b + 32 + 32 * half + idx) >> (2 * j)) & 0x03030303u;
            const uint32_t q1 = (gg_rd32<A2>(b + 36 + 32 * half + idx) >> (2 * j)) & 0x03030303u;
            const uint32_t m0 = ((gg_rd32<A2>(b + idx) >> hb) & 0x01010101u) ^ 0x01010101u;
            const uint32_t m1 = ((gg_rd32<A2>(b + idx + 4) >> hb) & 0x01010101u) ^ 0x01010101u;
            w0 = (int)(((q0 | 0x80808080u) - (m0 << 2)) ^ 0x80808080u);
            w1 = (int)(((q1 | 0x80808080u) - (m1 << 2)) ^ 0x80808080u);
            return;
        }
        case 12:
        case 13: {
            const int bb = t == 12 ? 144 : 176;
            const uint8_t* b = row + (size_t)(k / 256) * bb;
            const int p = k % 256, c64 = p / 64, c = p % 64, l0 = c % 32, hi = c / 32;
            const int js = 2 * c64 + hi;
            const uint8_t* s = b + 4;
            int sc, mn;
            if (js < 4) {
                sc = s[js] & 63;
                mn = s[js + 4] & 63;
            } else {
                sc = (s[js + 4] & 15) | ((s[js - 4] >> 6) << 4);
                mn = (s[js + 4] >> 4) | ((s[js] >> 6) << 4);
            }
            ds = gg_rdf16<A2>(b) * (float)sc;
            dm = gg_rdf16<A2>(b + 2) * (float)mn;
            const uint8_t* q = b + (t == 12 ? 16 : 48) + 32 * c64 + l0;
            uint32_t a0 = (gg_rd32<A2>(q) >> (4 * hi)) & 0x0f0f0f0fu;
            uint32_t a1 = (gg_rd32<A2>(q + 4) >> (4 * hi)) & 0x0f0f0f0fu;
            if (t == 13) {
                a0 |= ((gg_rd32<A2>(b + 16 + l0) >> js) & 0x01010101u) << 4;
                a1 |= ((gg_rd32<A2>(b + 20 + l0) >> js) & 0x01010101u) << 4;
            }
            w0 = (int)a0;
            w1 = (int)a1;
            return;
        }
        case 14: {
            const uint8_t* b = row + (size_t)(k / 256) * 210;
            const int p = k % 256, nn = p / 128, r = p % 128, quarter = r / 32, l0 = r % 32;
            const uint8_t* ql = b + 64 * nn + 32 * (quarter & 1) + l0;
            const uint8_t* qh = b + 128 + 32 * nn + l0;
            ds = gg_rdf16<A2>(b + 208) * (float)(int8_t)b[192 + 8 * nn + l0 / 16 + 2 * quarter];
            const int sl = 4 * (quarter >> 1), sh = 2 * quarter;
            // q6 - 32 per byte: (lo | hi << 4) in 0..63, minus 32 by a bytewise
            // subtract with no borrow across bytes (each byte >= 0, result -32..31).
            const uint32_t u0 = ((gg_rd32<A2>(ql) >> sl) & 0x0f0f0f0fu) |
                                (((gg_rd32<A2>(qh) >> sh) & 0x03030303u) << 4);
            const uint32_t u1 = ((gg_rd32<A2>(ql + 4) >> sl) & 0x0f0f0f0fu) |
                                (((gg_rd32<A2>(qh + 4) >> sh) & 0x03030303u) << 4);
            w0 = (int)((u0 | 0x80808080u) - 0x20202020u) ^ (int)0x80808080u;
            w1 = (int)((u1 | 0x80808080u) - 0x20202020u) ^ (int)0x80808080u;
            return;
        }
        case 18: {
            const uint8_t* b = row + (size_t)(k / 256) * 98;
            const int p = k % 256, ib = p / 32, l = (p % 32) / 8;
            const uint32_t aux = gg_rd32<A2>(b + 66 + 4 * ib);
            ds = gg_rdf16<A2>(b) * (0.5f + (float)(aux >> 28)) * 0.5f;
            const uint32_t i7 = (aux >> (7 * l)) & 127u;
            uint32_t n0, n1;
            if constexpr (A2) {
                const uint2 m = *reinterpret_cast<const uint2*>(sgn + 2 * i7);
                n0 = m.x;
                n1 = m.y;
            } else {
                const uint32_t signs = i7 | ((uint32_t)(__builtin_popcount(i7) & 1) << 7);
                n0 = gg_bytemask4(signs);
                n1 = gg_bytemask4(signs >> 4);
            }
            const uint32_t qs = A2 ? *reinterpret_cast<const uint16_t*>(b + 2 + 8 * ib + 2 * l)
                                   : (uint32_t)(b[2 + 8 * ib + 2 * l] | (b[3 + 8 * ib + 2 * l] << 8));
            const uint32_t g0 = grid[qs & 255u], g1 = grid[qs >> 8];
            // negate the flagged bytes: (g ^ 0xff) + 1 per byte, with no carry
            // out of a byte since every grid magnitude is at least 4
            w0 = (int)((g0 ^ n0) + (n0 & 0x01010101u));
            w1 = (int)((g1 ^ n1) + (n1 & 0x01010101u));
            return;
        }
        case 23: {
            const uint8_t* b = row + (size_t)(k / 256) * 136;
            const int p = k % 256, ib = p / 32, c = p % 32;
            const int sh = A2 ? *reinterpret_cast<const uint16_t*>(b + 2) : (b[2] | (b[3] << 8));
            const int lo = (b[4 + ib / 2] >> (4 * (ib & 1))) & 15;
            const int hi = (sh >> (2 * ib)) & 3;
            ds = gg_rdf16<A2>(b) * (float)((int)(int8_t)(uint8_t)(lo | (hi << 4)) - 32);
            const uint8_t* q = b + 8 + 16 * ib + (c % 16);
            const int shq = 4 * (c / 16);
            w0 = (int)gg_iq4nl4((gg_rd32<A2>(q) >> shq) & 0x0f0f0f0fu);
            w1 = (int)gg_iq4nl4((gg_rd32<A2>(q + 4) >> shq) & 0x0f0f0f0fu);
            return;
        }
        default:
            ds = 0.0f;
            w0 = w1 = 0;
            return;
    }
}

template <uint32_t T, bool A2 = false>
__device__ __forceinline__ void gg_dec8i(uint32_t t, const uint8_t* __restrict__ row, int k,
                                         const uint32_t* __restrict__ grid,
                                         const uint32_t* __restrict__ sgn, int& w0, int& w1,
                                         float& ds, float& dm) {
    gg_dec8i_any<A2>(T == kGgAny ? t : T, row, k, grid, sgn, w0, w1, ds, dm);
}

// LDS tile of int8 activations: TT rows x kGgKC bytes and their per-32 scales.
template <int TT>
struct GgI8Tile {
    int q[TT][kGgKC / 4];
    float s[TT][kGgKC / 32];
};

// The int8 twin of gg_dots: xq [*, K] int8 and xsc [*, K / 32] scales; per
// 8-element fragment r = ds * dot(wq, xq) - dm * sum(xq), acc += sx * r.
template <uint32_t T, int NM, int TT>
__device__ __forceinline__ void gg_dots_i8(GgI8Tile<TT>& xt, int* srcs, const int8_t* __restrict__ xq,
                                           const float* __restrict__ xsc, int K,
                                           const GgTile<TT>& tl, const uint32_t (&type)[NM],
                                           const uint8_t* const (&wrow)[NM][4],
                                           float (&acc)[NM][4][TT]) {
    const int lane = threadIdx.x & 63;
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int t = 0; t < TT; ++t) srcs[t] = tl.src[t];
    }
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int t = 0; t < TT; ++t) acc[m][r][t] = 0.0f;
    const int K32 = K / 32;
    for (int k0 = 0; k0 < K; k0 += kGgKC) {
        const int kc = min(kGgKC, K - k0);
        __syncthreads();
        for (int i = threadIdx.x; i < TT * (kGgKC / 4); i += blockDim.x) {
            const int t = i / (kGgKC / 4), c = i % (kGgKC / 4);
            int v = 0;
            if (t < tl.nr && 4 * c < kc)
                v = *reinterpret_cast<const int*>(xq + (size_t)srcs[t] * K + k0 + 4 * c);
            xt.q[t][c] = v;
        }
        for (int i = threadIdx.x; i < TT * (kGgKC / 32); i += blockDim.x) {
            const int t = i / (kGgKC / 32), c = i % (kGgKC / 32);
            xt.s[t][c] = (t < tl.nr && 32 * c < kc) ? xsc[(size_t)srcs[t] * K32 + k0 / 32 + c] : 0.0f;
        }
        __syncthreads();
        const int kk = lane * 8;
        if (kk >= kc) continue;
        int x0[TT], x1[TT], sx1[TT];
        float sx[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const int2 q = *reinterpret_cast<const int2*>(&xt.q[t][kk / 4]);
            x0[t] = q.x;
            x1[t] = q.y;
            sx[t] = xt.s[t][kk / 32];
            sx1[t] = __builtin_amdgcn_sdot4(0x01010101, q.y, __builtin_amdgcn_sdot4(0x01010101, q.x, 0, false), false);
        }
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                int w0, w1;
                float ds, dm;
                gg_dec8i<T>(type[m], wrow[m][r], k0 + kk, c_iq3xxs_grid, nullptr, w0, w1, ds, dm);
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    const int si = __builtin_amdgcn_sdot4(w1, x1[t], __builtin_amdgcn_sdot4(w0, x0[t], 0, false), false);
                    float v = ds * (float)si;
                    if (T == 12 || T == 13 || (T == kGgAny && dm != 0.0f)) v = v - dm * (float)sx1[t];
                    acc[m][r][t] = __builtin_fmaf(sx[t], v, acc[m][r][t]);
                }
            }
    }
}

// ---- Streamed weights (the block types, one type per matrix set). Each wave
// owns 4 weight rows per matrix; per K chunk it loads those rows' block bytes
// with coalesced dword loads (lane l: dwords l, l + 64, ...) one chunk ahead
// into registers, parks them in a private LDS buffer and decodes from there,
// so every weight byte is one wide load and a chunk is in flight while the
// previous one is decoded. The tile's activations are staged the same way
// (shared by the four waves, one barrier per chunk).
constexpr int gg_be(uint32_t t) { return t == 8 ? 32 : 256; }
constexpr int gg_bb(uint32_t t) {
    return t == 8 ? 34 : t == 11 ? 110 : t == 12 ? 144 : t == 13 ? 176 : t == 14 ? 210
         : t == 18 ? 98 : t == 23 ? 136 : 0;
}
// K per chunk: at most 3 dwords per lane per row, and 512 for 8-row tiles (LDS).
// Lane l always takes K elements 512 f + 8 l of each 512, so the sums do not
// depend on the chunk size.
constexpr int gg_kc(uint32_t t, int tt) { return (t == 8 || t == 14 || tt > 1) ? 512 : 1024; }
constexpr bool gg_streamed(uint32_t t) { return gg_bb(t) != 0; }

template <uint32_t T, int NM, int TT, bool I8>
struct GgStream {
    static constexpr int KC = gg_kc(T, TT);
    static constexpr int CB = KC / gg_be(T) * gg_bb(T);   // bytes of a row's chunk
    static constexpr int ND = CB / 4;
    static constexpr int LPR = (ND + 63) / 64;            // dword loads per lane per row
    static constexpr int XV = I8 ? TT * KC / 4 : TT * KC / 4;   // int / float4 items of x
    static constexpr int XR = (XV + kGgThreads - 1) / kGgThreads;   // per thread
    static constexpr int SR = TT * KC / 32;               // scales (I8)
    uint32_t w[2][kGgWaves][NM * 4][ND];
    uint32_t grid[T == 18 ? 256 : 1];   // the IQ3_XXS codebook
    uint32_t sgn[T == 18 ? 256 : 1];    // IQ3_XXS: byte masks of the 128 sign patterns
    float x[I8 ? 1 : 2][I8 ? 1 : TT][I8 ? 4 : KC];
    struct {
        int q[I8 ? 2 : 1][I8 ? TT : 1][I8 ? KC / 4 : 1];
        float s[I8 ? 2 : 1][I8 ? TT : 1][I8 ? KC / 32 : 1];
    } i8;
};

template <uint32_t T, int NM, int TT, bool I8>
__device__ __forceinline__ void gg_dots_stream(GgStream<T, NM, TT, I8>& L, int* srcs,
                                               const float* __restrict__ x,
                                               const int8_t* __restrict__ xq,
                                               const float* __restrict__ xsc, int K,
                                               const GgTile<TT>& tl,
                                               const uint8_t* const (&wrow)[NM][4],
                                               float (&acc)[NM][4][TT]) {
    using S = GgStream<T, NM, TT, I8>;
    constexpr int KC = S::KC, ND = S::ND, LPR = S::LPR, XR = S::XR;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tid = threadIdx.x;
    __syncthreads();   // srcs and the buffers of a previous tile are consumed
    if (tid == 0) {
#pragma unroll
        for (int t = 0; t < TT; ++t) srcs[t] = tl.src[t];
    }
    if constexpr (T == 18) {
        if (tid < 256) {
            L.grid[tid] = c_iq3xxs_grid[tid];
            // pattern e: 7 sign bits plus their parity bit, as 8 byte masks
            const uint32_t e = (uint32_t)tid >> 1;
            const uint32_t sg = e | ((uint32_t)(__builtin_popcount(e) & 1) << 7);
            L.sgn[tid] = gg_bytemask4(sg >> (4 * (tid & 1)));
        }
    }
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int t = 0; t < TT; ++t) acc[m][r][t] = 0.0f;
    __syncthreads();
    const int nch = (K + KC - 1) / KC;
    const int rowb = K / gg_be(T) * gg_bb(T);   // block bytes of a whole row
    uint32_t wr[NM * 4][LPR];
    float4 xr[XR];
    int qr[XR];
    float sr = 0.0f;
    auto load = [&](int c) {
        const int k0 = c * KC, kc = min(KC, K - k0);
        const int nd = min(ND, (rowb - c * S::CB) / 4);
#pragma unroll
        for (int i = 0; i < NM * 4; ++i)
#pragma unroll
            for (int j = 0; j < LPR; ++j) {
                const int d = j * 64 + lane;
                if (d < nd)
                    wr[i][j] = *reinterpret_cast<const uint32_t*>(wrow[i / 4][i % 4] +
                                                                  (size_t)c * S::CB + 4 * d);
            }
#pragma unroll
        for (int j = 0; j < XR; ++j) {
            const int v = tid + kGgThreads * j;
            const int t = v / (KC / 4), c4 = v % (KC / 4);
            if (v < S::XV && t < tl.nr && 4 * c4 < kc) {
                if constexpr (I8)
                    qr[j] = *reinterpret_cast<const int*>(xq + (size_t)srcs[t] * K + k0 + 4 * c4);
                else
                    xr[j] = *reinterpret_cast<const float4*>(x + (size_t)srcs[t] * K + k0 + 4 * c4);
            }
        }
        if constexpr (I8) {
            if (tid < S::SR) {
                const int t = tid / (KC / 32), c32 = tid % (KC / 32);
                sr = (t < tl.nr && 32 * c32 < kc)
                         ? xsc[(size_t)srcs[t] * (K / 32) + k0 / 32 + c32] : 0.0f;
            }
        }
    };
    auto park = [&](int b, int c) {
        const int k0 = c * KC, kc = min(KC, K - k0);
        const int nd = min(ND, (rowb - c * S::CB) / 4);
#pragma unroll
        for (int i = 0; i < NM * 4; ++i)
#pragma unroll
            for (int j = 0; j < LPR; ++j) {
                const int d = j * 64 + lane;
                if (d < nd) L.w[b][wave][i][d] = wr[i][j];
            }
#pragma unroll
        for (int j = 0; j < XR; ++j) {
            const int v = tid + kGgThreads * j;
            const int t = v / (KC / 4), c4 = v % (KC / 4);
            if (v < S::XV) {
                const bool ok = t < tl.nr && 4 * c4 < kc;
                if constexpr (I8)
                    L.i8.q[b][t][c4] = ok ? qr[j] : 0;
                else
                    *reinterpret_cast<float4*>(&L.x[b][t][4 * c4]) =
                        ok ? xr[j] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        if constexpr (I8) {
            if (tid < S::SR) L.i8.s[b][tid / (KC / 32)][tid % (KC / 32)] = sr;
        }
    };
    load(0);
    park(0, 0);
    __syncthreads();
    for (int c = 0; c < nch; ++c) {
        const int b = c & 1;
        if (c + 1 < nch) load(c + 1);
        const int kc = min(KC, K - c * KC);
#pragma unroll
        for (int f = 0; f < KC / 512; ++f) {
            const int kk = f * 512 + lane * 8;
            if (kk < kc) {
                if constexpr (I8) {
                    int x0[TT], x1[TT], sx1[TT];
                    float sx[TT];
#pragma unroll
                    for (int t = 0; t < TT; ++t) {
                        const int2 q = *reinterpret_cast<const int2*>(&L.i8.q[b][t][kk / 4]);
                        x0[t] = q.x;
                        x1[t] = q.y;
                        sx[t] = L.i8.s[b][t][kk / 32];
                        sx1[t] = __builtin_amdgcn_sdot4(
                            0x01010101, q.y, __builtin_amdgcn_sdot4(0x01010101, q.x, 0, false),
                            false);
                    }
#pragma unroll
                    for (int i = 0; i < NM * 4; ++i) {
                        int w0, w1;
                        float ds, dm;
                        gg_dec8i<T, true>(T, reinterpret_cast<const uint8_t*>(L.w[b][wave][i]),
                                          kk, L.grid, L.sgn, w0, w1, ds, dm);
#pragma unroll
                        for (int t = 0; t < TT; ++t) {
                            const int si = __builtin_amdgcn_sdot4(
                                w1, x1[t], __builtin_amdgcn_sdot4(w0, x0[t], 0, false), false);
                            float v = ds * (float)si;
                            if (T == 12 || T == 13) v = v - dm * (float)sx1[t];
                            acc[i / 4][i % 4][t] = __builtin_fmaf(sx[t], v, acc[i / 4][i % 4][t]);
                        }
                    }
                } else {
                    // The integer fragment (weight = ds * wq - dm, the reference's
                    // dequantized value exactly), then
                    // acc += ds * sum(wq * x) - dm * sum(x).
                    float xv[TT][8], sx[TT];
#pragma unroll
                    for (int t = 0; t < TT; ++t) {
                        const float4 a = *reinterpret_cast<const float4*>(&L.x[b][t][kk]);
                        const float4 e = *reinterpret_cast<const float4*>(&L.x[b][t][kk + 4]);
                        xv[t][0] = a.x; xv[t][1] = a.y; xv[t][2] = a.z; xv[t][3] = a.w;
                        xv[t][4] = e.x; xv[t][5] = e.y; xv[t][6] = e.z; xv[t][7] = e.w;
                        if (T == 12 || T == 13) {
                            float v = xv[t][0];
#pragma unroll
                            for (int j = 1; j < 8; ++j) v = v + xv[t][j];
                            sx[t] = v;
                        }
                    }
#pragma unroll
                    for (int i = 0; i < NM * 4; ++i) {
                        int w0, w1;
                        float ds, dm;
                        gg_dec8i<T, true>(T, reinterpret_cast<const uint8_t*>(L.w[b][wave][i]),
                                          kk, L.grid, L.sgn, w0, w1, ds, dm);
                        float wf[8];
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            wf[j] = (float)(int8_t)((uint32_t)(j < 4 ? w0 : w1) >> (8 * (j & 3)));
#pragma unroll
                        for (int t = 0; t < TT; ++t) {
                            float v = wf[0] * xv[t][0];
#pragma unroll
                            for (int j = 1; j < 8; ++j) v = __builtin_fmaf(wf[j], xv[t][j], v);
                            float& ac = acc[i / 4][i % 4][t];
                            ac = __builtin_fmaf(ds, v, ac);
                            if (T == 12 || T == 13) ac = __builtin_fmaf(-dm, sx[t], ac);
                        }
                    }
                }
            }
        }
        if (c + 1 < nch) park(b ^ 1, c + 1);
        __syncthreads();
    }
}

// quantize_act_q8 (cuda/qgemm.cu:556-587): per 32-element block (one half
// wave), sx = absmax / 127, q = round-half-even(v * (1 / sx)), 0 when sx = 0.
__global__ __launch_bounds__(256) void gg_quant_q8_kernel(const float* __restrict__ x, long total,
                                                          int8_t* __restrict__ xq,
                                                          float* __restrict__ xs) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const float v = i < total ? x[i] : 0.0f;
    float a = fabsf(v);
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) a = fmaxf(a, __shfl_xor(a, m));
    if (i >= total) return;
    const float sx = a / 127.0f;
    const float id = sx > 0.0f ? 1.0f / sx : 0.0f;
    xq[i] = (int8_t)(int)rintf(v * id);
    if ((i & 31) == 0) xs[i / 32] = sx;
}

// gemm_q: tiles are 8 consecutive tokens (one at n = 1), one tile per
// workgroup row of the grid.
// LDS bytes of a tile's staged activations.
template <int TT, bool I8>
constexpr size_t gg_lds_bytes() {
    return I8 ? sizeof(GgI8Tile<TT>) : sizeof(float) * TT * kGgKC;
}

// I8: activations are (xq, xsc) from quantize_act_q8 instead of x (gemm_q_i8).
template <uint32_t T, int TT, bool I8>
__global__ __launch_bounds__(kGgThreads) void gg_gemv_kernel(uint32_t qtype, const float* __restrict__ x,
                                                      const int8_t* __restrict__ xq,
                                                      const float* __restrict__ xsc,
                                                      const uint8_t* __restrict__ qw,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ y, int n, int in, int out,
                                                      long row_bytes) {
    constexpr bool ST = gg_streamed(T);
    __shared__ __align__(16) char lds[ST ? sizeof(GgStream<T, 1, TT, I8>) : gg_lds_bytes<TT, I8>()];
    __shared__ int srcs[TT];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int o0 = blockIdx.x * kGgRows + wave * 4;
    const uint32_t type[1] = {qtype};
    const uint8_t* wrow[1][4];
#pragma unroll
    for (int r = 0; r < 4; ++r) wrow[0][r] = qw + (size_t)min(o0 + r, out - 1) * row_bytes;
    // token tiles: blockIdx.y, then strided by the grid's height
    for (int t0 = blockIdx.y * TT; t0 < n; t0 += gridDim.y * TT) {
        GgTile<TT> tl;
        tl.e = 0;
        tl.nr = min(TT, n - t0);
#pragma unroll
        for (int t = 0; t < TT; ++t) tl.row[t] = tl.src[t] = min(t0 + t, n - 1);
        float acc[1][4][TT];
        if constexpr (ST)
            gg_dots_stream<T, 1, TT, I8>(*reinterpret_cast<GgStream<T, 1, TT, I8>*>(lds), srcs, x,
                                         xq, xsc, in, tl, wrow, acc);
        else if constexpr (I8)
            gg_dots_i8<T, 1, TT>(*reinterpret_cast<GgI8Tile<TT>*>(lds), srcs, xq, xsc, in, tl, type,
                                 wrow, acc);
        else
            gg_dots<T, 1, TT>(reinterpret_cast<float (*)[kGgKC]>(lds), srcs, x, in, tl, type, wrow,
                              acc);
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const float v = gg_wave_sum(acc[0][r][t]);
                const int o = o0 + r;
                if (lane == 0 && t < tl.nr && o < out)
                    y[(size_t)(t0 + t) * out + o] = bias ? v + bias[o] : v;
            }
    }
}

// Tile g of the routed rows. grouped: d = [offsets E+1 | tile prefix E+1 |
// rows n*topk] from gg_group_kernel; otherwise routed row g alone.
template <int TT>
__device__ __forceinline__ bool gg_tile(int g, const int* __restrict__ ids,
                                        const int* __restrict__ d, int nk, int E, int topk,
                                        bool down, GgTile<TT>& tl) {
    if (!d) {
        // An id outside [0, E) routes nowhere: no tile (the grouping drops it
        // too, and the reduce skips its slot).
        if (g >= nk || ids[g] < 0 || ids[g] >= E) return false;
        tl.e = ids[g];
        tl.nr = 1;
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            tl.row[t] = g;
            tl.src[t] = down ? g : g / topk;
        }
        return true;
    }
    const int* off = d;
    const int* tp = d + E + 1;
    const int* rows = d + 2 * (E + 1);
    if (g >= tp[E]) return false;
    int lo = 0, hi = E;   // the expert e with tp[e] <= g < tp[e + 1]
    while (hi - lo > 1) {
        const int mid = (lo + hi) / 2;
        if (tp[mid] <= g) lo = mid;
        else hi = mid;
    }
    tl.e = lo;
    const int r0 = off[lo] + (g - tp[lo]) * TT;
    tl.nr = min(TT, off[lo + 1] - r0);
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const int r = rows[r0 + (t < tl.nr ? t : 0)];
        tl.row[t] = r;
        tl.src[t] = down ? r : r / topk;
    }
    return true;
}

struct GgMoeArgs {
    uint32_t gate_type, up_type, down_type;
    const float* x;
    const int* ids;
    const float* w;
    const uint8_t *gate_q, *up_q, *down_q;
    long gate_rb, up_rb, down_rb;
    int n, topk, H, I, E;
    float* h_act;
    float* dpart;
    const int* d;   // grouping (nullable)
    // int8 activations (moe_expert_ffn_q_i8): x as (xq, xs), h_act as (hq, hs)
    const int8_t* xq;
    const float* xs;
    const int8_t* hq;
    const float* hs;
};

// DOWN = false: phase 1 (gate/up, output rows = I features); true: phase 2.
// T: the weight type (gate and up share it in phase 1), or kGgAny.
template <bool DOWN, uint32_t T, int TT, bool I8>
__global__ __launch_bounds__(kGgThreads) void gg_moe_kernel(GgMoeArgs a) {
    constexpr bool ST = gg_streamed(T);
    __shared__ __align__(16) char lds[ST ? sizeof(GgStream<T, DOWN ? 1 : 2, TT, I8>)
                                         : gg_lds_bytes<TT, I8>()];
    __shared__ int srcs[TT];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nk = a.n * a.topk;
    GgTile<TT> tl;
    if (!gg_tile((int)blockIdx.x, a.ids, a.d, nk, a.E, a.topk, DOWN, tl)) return;
    const int out = DOWN ? a.H : a.I;
    const int o0 = blockIdx.y * kGgRows + wave * 4;
    const size_t e = (size_t)tl.e;
    if constexpr (!DOWN) {
        const uint32_t type[2] = {a.gate_type, a.up_type};
        const uint8_t* wrow[2][4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const size_t o = (size_t)min(o0 + r, out - 1);
            wrow[0][r] = a.gate_q + (e * a.I + o) * a.gate_rb;
            wrow[1][r] = a.up_q + (e * a.I + o) * a.up_rb;
        }
        float acc[2][4][TT];
        if constexpr (ST)
            gg_dots_stream<T, 2, TT, I8>(*reinterpret_cast<GgStream<T, 2, TT, I8>*>(lds), srcs, a.x,
                                         a.xq, a.xs, a.H, tl, wrow, acc);
        else if constexpr (I8)
            gg_dots_i8<T, 2, TT>(*reinterpret_cast<GgI8Tile<TT>*>(lds), srcs, a.xq, a.xs, a.H, tl,
                                 type, wrow, acc);
        else
            gg_dots<T, 2, TT>(reinterpret_cast<float (*)[kGgKC]>(lds), srcs, a.x, a.H, tl, type,
                              wrow, acc);
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const float g = gg_wave_sum(acc[0][r][t]);
                const float u = gg_wave_sum(acc[1][r][t]);
                const int o = o0 + r;
                if (lane == 0 && t < tl.nr && o < out)
                    a.h_act[(size_t)tl.row[t] * a.I + o] = gg_silu(g) * u;
            }
    } else {
        const uint32_t type[1] = {a.down_type};
        const uint8_t* wrow[1][4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const size_t o = (size_t)min(o0 + r, out - 1);
            wrow[0][r] = a.down_q + (e * a.H + o) * a.down_rb;
        }
        float acc[1][4][TT];
        if constexpr (ST)
            gg_dots_stream<T, 1, TT, I8>(*reinterpret_cast<GgStream<T, 1, TT, I8>*>(lds), srcs,
                                         a.h_act, a.hq, a.hs, a.I, tl, wrow, acc);
        else if constexpr (I8)
            gg_dots_i8<T, 1, TT>(*reinterpret_cast<GgI8Tile<TT>*>(lds), srcs, a.hq, a.hs, a.I, tl,
                                 type, wrow, acc);
        else
            gg_dots<T, 1, TT>(reinterpret_cast<float (*)[kGgKC]>(lds), srcs, a.h_act, a.I, tl, type,
                              wrow, acc);
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const float v = gg_wave_sum(acc[0][r][t]);
                const int o = o0 + r;
                if (lane == 0 && t < tl.nr && o < out) a.dpart[(size_t)tl.row[t] * a.H + o] = v;
            }
    }
}

// out[t] = ((0 + w0 y0) + w1 y1) + ... over the slots (cuda/qgemm.cu:943-955).
// Slots whose id is outside [0, E) add nothing (their dpart rows are never
// written).
__global__ __launch_bounds__(256) void gg_reduce_kernel(const float* __restrict__ dpart,
                                                        const int* __restrict__ ids,
                                                        const float* __restrict__ w, int n,
                                                        int topk, int H, int E, float* __restrict__ out) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)n * H) return;
    const long t = i / H, o = i % H;
    float acc = 0.0f;
    for (int s = 0; s < topk; ++s) {
        const int e = ids[t * topk + s];
        if (e >= 0 && e < E) acc = acc + w[t * topk + s] * dpart[(t * topk + s) * H + o];
    }
    out[i] = acc;
}

// Groups the routed rows by expert (one workgroup): d = [offsets E+1 | tile
// prefix E+1 | rows n*topk]; rows of an expert are in any order (each row's
// result depends only on its own inputs).
__global__ __launch_bounds__(1024) void gg_group_kernel(const int* __restrict__ ids, int nk, int E,
                                                        int tile_rows, int* __restrict__ d) {
    extern __shared__ int gl[];   // cnt[E] | cursor[E]
    int* cnt = gl;
    int* cur = gl + E;
    int* off = d;
    int* tp = d + E + 1;
    int* rows = d + 2 * (E + 1);
    for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < nk; i += blockDim.x) {
        const int e = ids[i];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // Exclusive prefix sums of rows and tiles over the experts: thread i owns
    // experts [i * per, (i + 1) * per); a shuffle scan per wave, then the 16
    // wave totals.
    __shared__ int wsum[2][16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int per = (E + 1023) / 1024, e0 = min(E, tid * per), e1 = min(E, e0 + per);
    int o = 0, t = 0;
    for (int e = e0; e < e1; ++e) {
        o += cnt[e];
        t += (cnt[e] + tile_rows - 1) / tile_rows;
    }
    int so = o, st = t;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const int a = __shfl_up(so, m), b = __shfl_up(st, m);
        if (lane >= m) {
            so += a;
            st += b;
        }
    }
    if (lane == 63) {
        wsum[0][wave] = so;
        wsum[1][wave] = st;
    }
    __syncthreads();
    int bo = so - o, bt = st - t;
    for (int w = 0; w < wave; ++w) {
        bo += wsum[0][w];
        bt += wsum[1][w];
    }
    for (int e = e0; e < e1; ++e) {
        off[e] = bo;
        tp[e] = bt;
        cur[e] = bo;
        bo += cnt[e];
        bt += (cnt[e] + tile_rows - 1) / tile_rows;
    }
    if (tid == 1023) {
        off[E] = bo;
        tp[E] = bt;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nk; i += blockDim.x) {
        const int e = ids[i];
        if (e >= 0 && e < E) rows[atomicAdd(&cur[e], 1)] = i;
    }
}

// Calls f(std::integral_constant<uint32_t, t>) for a supported type t,
// f(kGgAny constant) otherwise.
template <class F>
static void gg_by_type(uint32_t t, F&& f) {
    switch (t) {
        case 0: f(std::integral_constant<uint32_t, 0>{}); break;
        case 1: f(std::integral_constant<uint32_t, 1>{}); break;
        case 8: f(std::integral_constant<uint32_t, 8>{}); break;
        case 11: f(std::integral_constant<uint32_t, 11>{}); break;
        case 12: f(std::integral_constant<uint32_t, 12>{}); break;
        case 13: f(std::integral_constant<uint32_t, 13>{}); break;
        case 14: f(std::integral_constant<uint32_t, 14>{}); break;
        case 18: f(std::integral_constant<uint32_t, 18>{}); break;
        case 23: f(std::integral_constant<uint32_t, 23>{}); break;
        default: f(std::integral_constant<uint32_t, kGgAny>{}); break;
    }
}

// The int8-capable types (qtype_has_i8, cuda/qgemm.cu:556-567).
bool gguf_has_i8(uint32_t t) {
    return t == 8 || t == 11 || t == 12 || t == 13 || t == 14 || t == 18 || t == 23;
}

// gg_by_type over the int8-capable types (kGgAny for anything else).
template <class F>
static void gg_by_type_i8(uint32_t t, F&& f) {
    switch (t) {
        case 8: f(std::integral_constant<uint32_t, 8>{}); break;
        case 11: f(std::integral_constant<uint32_t, 11>{}); break;
        case 12: f(std::integral_constant<uint32_t, 12>{}); break;
        case 13: f(std::integral_constant<uint32_t, 13>{}); break;
        case 14: f(std::integral_constant<uint32_t, 14>{}); break;
        case 18: f(std::integral_constant<uint32_t, 18>{}); break;
        case 23: f(std::integral_constant<uint32_t, 23>{}); break;
        default: f(std::integral_constant<uint32_t, kGgAny>{}); break;
    }
}

template <bool I8, class F>
static void gg_by_type_t(uint32_t t, F&& f) {
    if constexpr (I8) gg_by_type_i8(t, f);
    else gg_by_type(t, f);
}

// The streamed kernels load weight rows as dwords and fp32 activations as
// float4: with rows or bases not aligned for that, the type is decoded by the
// runtime switch (kGgAny) with byte loads instead.
static bool gg_aligned(const void* w, long row_bytes, const void* x, int xalign) {
    return ((uintptr_t)w & 3) == 0 && (row_bytes & 3) == 0 &&
           (x == nullptr || ((uintptr_t)x & (uintptr_t)(xalign - 1)) == 0);
}

template <bool I8>
static int gg_gemm(uint32_t qtype, const float* x, const int8_t* xq, const float* xsc,
                   const uint8_t* qw, const float* bias, float* y, int n, int in, int out,
                   long row_bytes, hipStream_t s) {
    const int tt = n == 1 ? 1 : 8;
    const dim3 grid((unsigned)((out + kGgRows - 1) / kGgRows),
                    (unsigned)std::min((n + tt - 1) / tt, 65535));
    const bool al = gg_aligned(qw, row_bytes, I8 ? (const void*)xq : (const void*)x, I8 ? 4 : 16);
    gg_by_type_t<I8>(al ? qtype : kGgAny, [&](auto tc) {
        constexpr uint32_t T = decltype(tc)::value;
        if (n == 1)
            hipLaunchKernelGGL((gg_gemv_kernel<T, 1, I8>), grid, dim3(kGgThreads), 0, s, qtype, x, xq,
                               xsc, qw, bias, y, n, in, out, row_bytes);
        else
            hipLaunchKernelGGL((gg_gemv_kernel<T, 8, I8>), grid, dim3(kGgThreads), 0, s, qtype, x, xq,
                               xsc, qw, bias, y, n, in, out, row_bytes);
    });
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_gg_gemm(uint32_t qtype, const float* x, const uint8_t* qw, const float* bias, float* y,
                   int n, int in, int out, long row_bytes, hipStream_t s) {
    return gg_gemm<false>(qtype, x, nullptr, nullptr, qw, bias, y, n, in, out, row_bytes, s);
}

int launch_gg_gemm_i8(uint32_t qtype, const int8_t* xq, const float* xs, const uint8_t* qw,
                      const float* bias, float* y, int n, int in, int out, long row_bytes,
                      hipStream_t s) {
    return gg_gemm<true>(qtype, nullptr, xq, xs, qw, bias, y, n, in, out, row_bytes, s);
}

int launch_gg_quant_q8(const float* x, long total, int8_t* xq, float* xs, hipStream_t s) {
    hipLaunchKernelGGL(gg_quant_q8_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       x, total, xq, xs);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// ---- Large groups on the matrix cores: moe_expert_ffn_q_i8 from
// kGgMmaMinRows routed rows, the reference's tensor-core policy
// (GLMSERVE_MMA_MOE_MIN_TS = 2048, cuda/qgemm.cu:1563-1587; its kernel
// emajor_mma_s8_kernel, :1262-1349). The arithmetic class is the reference's:
// per 32-element block an exact int32 dot of the int8 weights and int8
// activations, then * weight scale * activation scale added in fp32.
//
// Tiles: the routed rows grouped by expert (gg_group_kernel) in tiles of up
// to kGgMmaTM rows. A workgroup (8 waves) computes one tile x kGgMmaRows
// weight rows: phase 1 128 features (wave w: the gate rows and the up rows
// of features 16 w .. 16 w + 15, stacked as one 32-row block, so a lane
// holds gate and up of the same feature), phase 2 256 output rows (wave w:
// rows 32 w .. 32 w + 31). Per 256-K chunk:
//   - the chunk's raw block bytes of the workgroup's weight rows (IQ3_XXS,
//     IQ4_XS) and the tile's int8 activation rows and scales arrive in
//     registers, loaded one chunk ahead (coalesced: two threads per row);
//   - they are written to LDS; each thread decodes 4 of its row's 32-element
//     sub-blocks to int8 plus the sub-block's scale (the decode of
//     gg_dec8i_any per 32 elements: the scale read and computed once per
//     sub-block; the same float operations, so the same scale values);
//     Q8_0 sub-blocks are read from global memory directly;
//   - each wave runs v_mfma_i32_32x32x32_i8 per 32-block over its 32 weight
//     rows x the tile's 4 blocks of 32 rows (A = weights, B = activations:
//     a lane's 16 outputs are one row's 16 weight rows, so their 16 weight
//     scales come as 4 broadcast LDS reads and the row's activation scale
//     as one), then acc += (d * w_scale) * x_scale in fp32.
// Rows past the tile's end repeat its last row and are not stored; 32-row
// blocks wholly past it skip their MFMAs.
constexpr int kGgMmaMinRows = 2048;
constexpr int kGgMmaTM = 128;       // routed rows per tile
constexpr int kGgMmaRows = 256;     // weight rows per workgroup (8 waves x 32)
constexpr int kGgMmaStride = 272;   // LDS bytes per int8 row of a chunk (256 + 16 padding)
constexpr int kGgMmaThreads = 512;

typedef int gg_i32x4 __attribute__((ext_vector_type(4)));
typedef int gg_i32x16 __attribute__((ext_vector_type(16)));

// Raw chunk bytes of one row in LDS (IQ3_XXS 98, IQ4_XS 136; Q8_0 is decoded
// from global memory) and the per-thread register words that carry them.
template <uint32_t T>
struct GgMmaRaw {
    static constexpr int kBytes = T == 18 ? 98 : T == 23 ? 136 : 0;
    static constexpr int kStride = T == 18 ? 104 : T == 23 ? 144 : 16;
    // IQ3_XXS rows are 2-byte aligned: 16-bit pieces, 25 per thread; IQ4_XS
    // rows are 4-byte aligned: dwords, 17 per thread.
    static constexpr int kPiece = T == 18 ? 2 : 4;
    static constexpr int kPieces = kBytes / kPiece;
    static constexpr int kPerThread = (kPieces + 1) / 2;
};

template <uint32_t T>
struct GgMmaLds {
    int8_t wq[kGgMmaRows * kGgMmaStride];
    int8_t xq[kGgMmaTM * kGgMmaStride];
    float ws[8][kGgMmaRows];   // [32-block][weight row]
    float xs[8][kGgMmaTM];     // [32-block][tile row]
    uint8_t raw[kGgMmaRows * GgMmaRaw<T>::kStride];
    uint32_t grid[256];        // IQ3_XXS codebook
    uint32_t sgn[256];         // IQ3_XXS sign byte masks, two words per 7-bit pattern
    int src[kGgMmaTM];         // activation row of each tile row
    int row[kGgMmaTM];         // routed row of each tile row
};

// Bytes of one 256-element chunk of a row of type T.
__host__ __device__ constexpr int gg_mma_chunk_bytes(uint32_t t) {
    return t == 18 ? 98 : t == 23 ? 136 : t == 8 ? 8 * 34 : 0;
}
bool gg_mma_type_ok(uint32_t t) { return t == 8 || t == 18 || t == 23; }

// Sub-block ib (32 elements) of a chunk as 8 int8 words plus its scale.
// IQ3_XXS / IQ4_XS from the LDS copy of the chunk (b), Q8_0 from global (g).
template <uint32_t T>
__device__ __forceinline__ void gg_mma_sub(const uint8_t* b, const uint8_t* g, int ib,
                                           const uint32_t* grid, const uint32_t* sgn, uint32_t (&w)[8],
                                           float& ds) {
    if constexpr (T == 18) {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(b);
        const uint32_t aux = (uint32_t)h[33 + 2 * ib] | ((uint32_t)h[34 + 2 * ib] << 16);
        ds = (float)__builtin_bit_cast(_Float16, h[0]) * (0.5f + (float)(aux >> 28)) * 0.5f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t i7 = (aux >> (7 * l)) & 127u;
            const uint2 m = *reinterpret_cast<const uint2*>(sgn + 2 * i7);
            const uint32_t qs = h[1 + 4 * ib + l];
            const uint32_t g0 = grid[qs & 255u], g1 = grid[qs >> 8];
            w[2 * l] = (g0 ^ m.x) + (m.x & 0x01010101u);
            w[2 * l + 1] = (g1 ^ m.y) + (m.y & 0x01010101u);
        }
    } else if constexpr (T == 23) {
        const uint16_t sh = *reinterpret_cast<const uint16_t*>(b + 2);
        const int lo = (b[4 + ib / 2] >> (4 * (ib & 1))) & 15;
        const int hi = (sh >> (2 * ib)) & 3;
        ds = (float)__builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t*>(b)) *
             (float)((int)(int8_t)(uint8_t)(lo | (hi << 4)) - 32);
        const uint2 q01 = *reinterpret_cast<const uint2*>(b + 8 + 16 * ib);
        const uint2 q23 = *reinterpret_cast<const uint2*>(b + 16 + 16 * ib);
        const uint32_t q[4] = {q01.x, q01.y, q23.x, q23.y};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            w[j] = gg_iq4nl4(q[j] & 0x0f0f0f0fu);
            w[4 + j] = gg_iq4nl4((q[j] >> 4) & 0x0f0f0f0fu);
        }
    } else {   // Q8_0: block ib of the chunk (34 bytes, 2-byte aligned) in global memory
        const uint16_t* h = reinterpret_cast<const uint16_t*>(g + 34 * ib);
        ds = (float)__builtin_bit_cast(_Float16, h[0]);
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = (uint32_t)h[1 + 2 * j] | ((uint32_t)h[2 + 2 * j] << 16);
    }
}

template <bool DOWN, uint32_t T>
__global__ __launch_bounds__(kGgMmaThreads) void gg_mma_kernel(GgMoeArgs a) {
    using RW = GgMmaRaw<T>;
    __shared__ __align__(16) GgMmaLds<T> L;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int E = a.E;
    const int* off = a.d;
    const int* tp = a.d + E + 1;
    const int* rows = a.d + 2 * (E + 1);
    const int g = (int)blockIdx.x;
    if (g >= tp[E]) return;   // the grid covers the largest possible tile count
    int lo = 0, hi = E;       // the expert e with tp[e] <= g < tp[e + 1]
    while (hi - lo > 1) {
        const int mid = (lo + hi) / 2;
        if (tp[mid] <= g) lo = mid;
        else hi = mid;
    }
    const int e = lo;
    const int r0 = off[e] + (g - tp[e]) * kGgMmaTM;
    const int nr = min(kGgMmaTM, off[e + 1] - r0);
    if (tid < kGgMmaTM) {
        const int r = rows[r0 + min(tid, nr - 1)];
        L.row[tid] = r;
        L.src[tid] = DOWN ? r : r / a.topk;
    }
    if constexpr (T == 18) {
        if (tid < 256) {
            L.grid[tid] = c_iq3xxs_grid[tid];
            const uint32_t pe = (uint32_t)tid >> 1;
            const uint32_t sg = pe | ((uint32_t)(__builtin_popcount(pe) & 1) << 7);
            L.sgn[tid] = gg_bytemask4(sg >> (4 * (tid & 1)));
        }
    }
    const int K = DOWN ? a.I : a.H;
    const int nch = K / 256;
    constexpr int CB = gg_mma_chunk_bytes(T);
    // This thread stages and decodes half (sub-blocks 4 fh .. 4 fh + 3) of
    // weight row rr of the workgroup.
    const int rr = tid >> 1, fh = tid & 1;
    const uint8_t* wrow;
    if constexpr (DOWN) {
        const size_t o = (size_t)blockIdx.y * kGgMmaRows + rr;
        wrow = a.down_q + ((size_t)e * a.H + o) * a.down_rb;
    } else {
        const int j = rr & 31;
        const size_t f = (size_t)blockIdx.y * 128 + 16 * (rr >> 5) + (j & 15);
        wrow = j < 16 ? a.gate_q + ((size_t)e * a.I + f) * a.gate_rb : a.up_q + ((size_t)e * a.I + f) * a.up_rb;
    }
    __syncthreads();
    const int8_t* X = DOWN ? a.hq : a.xq;
    const float* XS = DOWN ? a.hs : a.xs;
    // Activations: this thread stages 64 B (a quarter) of tile row xr's chunk
    // and (tid < 256) half of row tid / 2's 8 block scales.
    const int xr = tid >> 2, xqtr = tid & 3;
    const int8_t* xrow = X + (size_t)L.src[xr] * K + xqtr * 64;
    const float* xsrow = XS + (size_t)L.src[(tid >> 1) & (kGgMmaTM - 1)] * (K / 32) + 4 * (tid & 1);

    // The next chunk's loads (registers).
    uint32_t rv[RW::kPerThread > 0 ? RW::kPerThread : 1];
    uint4 xv0, xv1, xv2, xv3;
    float4 sv = make_float4(0.f, 0.f, 0.f, 0.f);
#define GG_MMA_LOAD(cc)                                                                              \
    do {                                                                                             \
        if constexpr (RW::kBytes > 0) {                                                              \
            const uint8_t* src_ = wrow + (size_t)(cc) * CB;                                          \
            _Pragma("unroll") for (int i = 0; i < RW::kPerThread; ++i) {                             \
                const int p = fh * RW::kPerThread + i;                                               \
                if (p < RW::kPieces) {                                                               \
                    if constexpr (RW::kPiece == 2) rv[i] = reinterpret_cast<const uint16_t*>(src_)[p]; \
                    else rv[i] = reinterpret_cast<const uint32_t*>(src_)[p];                         \
                }                                                                                    \
            }                                                                                        \
        }                                                                                            \
        const uint4* xp_ = reinterpret_cast<const uint4*>(xrow + (size_t)(cc) * 256);                \
        xv0 = xp_[0]; xv1 = xp_[1]; xv2 = xp_[2]; xv3 = xp_[3];                                      \
        if (tid < 2 * kGgMmaTM) sv = *reinterpret_cast<const float4*>(xsrow + (cc) * 8);             \
    } while (0)

    float acc[4][16];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[tb][i] = 0.0f;
    const int ar = wave * 32 + (lane & 31), hh = lane >> 5;
    // 32-row blocks of the tile holding rows: an expert's last tile (at
    // prefill sizes often its only one) skips the MFMAs of the empty blocks.
    const int ntb = __builtin_amdgcn_readfirstlane((nr + 31) / 32);
    GG_MMA_LOAD(0);
    for (int c = 0; c < nch; ++c) {
        // Stage chunk c.
        if constexpr (RW::kBytes > 0) {
#pragma unroll
            for (int i = 0; i < RW::kPerThread; ++i) {
                const int p = fh * RW::kPerThread + i;
                if (p < RW::kPieces) {
                    if constexpr (RW::kPiece == 2)
                        reinterpret_cast<uint16_t*>(L.raw + rr * RW::kStride)[p] = (uint16_t)rv[i];
                    else
                        reinterpret_cast<uint32_t*>(L.raw + rr * RW::kStride)[p] = rv[i];
                }
            }
        }
        {
            uint4* xd = reinterpret_cast<uint4*>(L.xq + xr * kGgMmaStride + xqtr * 64);
            xd[0] = xv0; xd[1] = xv1; xd[2] = xv2; xd[3] = xv3;
        }
        if (tid < 2 * kGgMmaTM) {
            const int t = tid >> 1, b0 = 4 * (tid & 1);
            L.xs[b0][t] = sv.x; L.xs[b0 + 1][t] = sv.y; L.xs[b0 + 2][t] = sv.z; L.xs[b0 + 3][t] = sv.w;
        }
        __syncthreads();
        // The next chunk (the last one again at the end: harmless reloads)
        // in flight during the decode and the MFMAs.
        GG_MMA_LOAD(c + 1 < nch ? c + 1 : c);
        // Decode this thread's 4 sub-blocks.
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int ib = 4 * fh + s;
            uint32_t w[8];
            float ds;
            gg_mma_sub<T>(L.raw + rr * RW::kStride, wrow + (size_t)c * CB, ib, L.grid, L.sgn, w, ds);
            uint4* dst = reinterpret_cast<uint4*>(L.wq + rr * kGgMmaStride + 32 * ib);
            dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
            dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
            L.ws[ib][rr] = ds;
        }
        __syncthreads();
#pragma unroll 2
        for (int kb = 0; kb < 8; ++kb) {
            const gg_i32x4 A = *reinterpret_cast<const gg_i32x4*>(L.wq + ar * kGgMmaStride + kb * 32 + hh * 16);
            float wsv[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = *reinterpret_cast<const float4*>(&L.ws[kb][wave * 32 + 8 * q + 4 * hh]);
                wsv[4 * q] = v.x; wsv[4 * q + 1] = v.y; wsv[4 * q + 2] = v.z; wsv[4 * q + 3] = v.w;
            }
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                if (tb < ntb) {   // blocks past the tile's rows skip (uniform)
                    const int xrow_l = tb * 32 + (lane & 31);
                    const gg_i32x4 B =
                        *reinterpret_cast<const gg_i32x4*>(L.xq + xrow_l * kGgMmaStride + kb * 32 + hh * 16);
                    const gg_i32x16 d = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, gg_i32x16{}, 0, 0, 0);
                    const float xsv = L.xs[kb][xrow_l];
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        acc[tb][i] = __builtin_fmaf((float)d[i] * wsv[i], xsv, acc[tb][i]);
                }
            }
        }
        __syncthreads();
    }
    // Lane: tile row tb * 32 + lane % 32; its 16 outputs are weight rows
    // 8 (i / 4) + 4 hh + i % 4 of the wave's 32-row block.
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
        const int t = tb * 32 + (lane & 31);
        if (t >= nr) continue;
        const size_t r = (size_t)L.row[t];
        if constexpr (DOWN) {
            float* dst = a.dpart + r * a.H + (size_t)blockIdx.y * kGgMmaRows + wave * 32 + 4 * hh;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<float4*>(dst + 8 * q) =
                    make_float4(acc[tb][4 * q], acc[tb][4 * q + 1], acc[tb][4 * q + 2], acc[tb][4 * q + 3]);
        } else {
            // i < 8: gate of feature 8 (i / 4) + 4 hh + i % 4; i + 8: its up.
            float* dst = a.h_act + r * a.I + (size_t)blockIdx.y * 128 + wave * 16 + 4 * hh;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                float hv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) hv[u] = gg_silu(acc[tb][4 * q + u]) * acc[tb][4 * q + u + 8];
                *reinterpret_cast<float4*>(dst + 8 * q) = make_float4(hv[0], hv[1], hv[2], hv[3]);
            }
        }
    }
}

#undef GG_MMA_LOAD

// The matrix-core phases for a batch the caller grouped with kGgMmaTM-row
// tiles; h_act is requantized into (hq, hs) between them.
static int gg_mma_phases(const GgMoeArgs& a, hipStream_t s) {
    const unsigned tiles = (unsigned)(a.n * a.topk / kGgMmaTM + a.E);
    auto by = [&](uint32_t t, auto f) {
        if (t == 8) f(std::integral_constant<uint32_t, 8>{});
        else if (t == 18) f(std::integral_constant<uint32_t, 18>{});
        else f(std::integral_constant<uint32_t, 23>{});
    };
    by(a.gate_type, [&](auto tc) {
        hipLaunchKernelGGL((gg_mma_kernel<false, decltype(tc)::value>), dim3(tiles, (unsigned)(a.I / 128)),
                           dim3(kGgMmaThreads), 0, s, a);
    });
    if (hipGetLastError() != hipSuccess) return -4;
    if (launch_gg_quant_q8(a.h_act, (long)a.n * a.topk * a.I, const_cast<int8_t*>(a.hq),
                           const_cast<float*>(a.hs), s))
        return -4;
    by(a.down_type, [&](auto tc) {
        hipLaunchKernelGGL((gg_mma_kernel<true, decltype(tc)::value>),
                           dim3(tiles, (unsigned)(a.H / kGgMmaRows)), dim3(kGgMmaThreads), 0, s, a);
    });
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// I8: h_act is quantized into (hq, hs) between the phases.
template <int TT, bool I8>
static int gg_moe_phases(uint32_t gt, uint32_t ut, uint32_t dt, const GgMoeArgs& a, unsigned tiles,
                         hipStream_t s) {
    const dim3 g1(tiles, (unsigned)((a.I + kGgRows - 1) / kGgRows));
    const bool al1 = gg_aligned(a.gate_q, a.gate_rb, I8 ? (const void*)a.xq : (const void*)a.x,
                                I8 ? 4 : 16) &&
                     gg_aligned(a.up_q, a.up_rb, nullptr, 1);
    const bool al2 = gg_aligned(a.down_q, a.down_rb,
                                I8 ? (const void*)a.hq : (const void*)a.h_act, I8 ? 4 : 16);
    if (gt == ut && al1)
        gg_by_type_t<I8>(gt, [&](auto tc) {
            hipLaunchKernelGGL((gg_moe_kernel<false, decltype(tc)::value, TT, I8>), g1, dim3(kGgThreads),
                               0, s, a);
        });
    else
        hipLaunchKernelGGL((gg_moe_kernel<false, kGgAny, TT, I8>), g1, dim3(kGgThreads), 0, s, a);
    if (hipGetLastError() != hipSuccess) return -4;
    if constexpr (I8) {
        if (launch_gg_quant_q8(a.h_act, (long)a.n * a.topk * a.I, const_cast<int8_t*>(a.hq),
                               const_cast<float*>(a.hs), s))
            return -4;
    }
    const dim3 g2(tiles, (unsigned)((a.H + kGgRows - 1) / kGgRows));
    gg_by_type_t<I8>(al2 ? dt : kGgAny, [&](auto tc) {
        hipLaunchKernelGGL((gg_moe_kernel<true, decltype(tc)::value, TT, I8>), g2, dim3(kGgThreads), 0, s,
                           a);
    });
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

template <bool I8>
static int gg_moe(GgMoeArgs a, float* out, int* dispatch, hipStream_t s) {
    const uint32_t gt = a.gate_type, ut = a.up_type, dt = a.down_type;
    const int n = a.n, topk = a.topk, H = a.H, E = a.E;
    const float* ids_w = a.w;
    const float* dpart = a.dpart;
    const int* ids = a.ids;
    const int nk = n * topk;
    // Rows per tile: about the rows an expert holds (decode: one or a few). With
    // one row per tile, grouping changes nothing but the order of the tiles, so
    // the routed rows are taken as they come (an exact grid, no counting pass).
    // int8 activations from kGgMmaMinRows routed rows, on types whose scale is
    // uniform over each 32-block and shapes of whole 256-K chunks: the
    // matrix-core phases (the reference's tensor-core policy).
    if constexpr (I8) {
        const bool al = ((uintptr_t)a.xq & 15) == 0 && ((uintptr_t)a.hq & 15) == 0 &&
                        ((uintptr_t)a.xs & 15) == 0 && ((uintptr_t)a.hs & 15) == 0 &&
                        ((uintptr_t)a.gate_q & 3) == 0 && ((uintptr_t)a.up_q & 3) == 0 &&
                        ((uintptr_t)a.down_q & 3) == 0 && (a.gate_rb & 3) == 0 && (a.up_rb & 3) == 0 &&
                        (a.down_rb & 3) == 0;
        if (dispatch && nk >= kGgMmaMinRows && gt == ut && gg_mma_type_ok(gt) && gg_mma_type_ok(dt) &&
            H % 256 == 0 && a.I % 256 == 0 && al) {
            hipLaunchKernelGGL(gg_group_kernel, dim3(1), dim3(1024), (size_t)2 * E * 4, s, ids, nk, E,
                               kGgMmaTM, dispatch);
            if (hipGetLastError() != hipSuccess) return -4;
            a.d = dispatch;
            const int rc = gg_mma_phases(a, s);
            if (rc) return rc;
            const long total = (long)n * H;
            hipLaunchKernelGGL(gg_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                               dpart, ids, ids_w, n, topk, H, E, out);
            return hipGetLastError() == hipSuccess ? 0 : -4;
        }
    }
    const int tt = !dispatch || nk <= E ? 1 : nk <= 4 * E ? 4 : 8;
    if (tt == 1) {
        dispatch = nullptr;
        a.d = nullptr;
    }
    unsigned tiles = (unsigned)nk;
    if (dispatch) {
        hipLaunchKernelGGL(gg_group_kernel, dim3(1), dim3(1024), (size_t)2 * E * 4, s, ids, nk, E,
                           tt, dispatch);
        if (hipGetLastError() != hipSuccess) return -4;
        tiles = (unsigned)((nk + tt - 1) / tt + E);
    }
    const int rc = tt == 1 ? gg_moe_phases<1, I8>(gt, ut, dt, a, tiles, s)
                 : tt == 4 ? gg_moe_phases<4, I8>(gt, ut, dt, a, tiles, s)
                           : gg_moe_phases<8, I8>(gt, ut, dt, a, tiles, s);
    if (rc) return rc;
    const long total = (long)n * H;
    hipLaunchKernelGGL(gg_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       dpart, ids, ids_w, n, topk, H, E, out);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_gg_moe(uint32_t gt, uint32_t ut, uint32_t dt, const float* x, const int* ids,
                  const float* w, const uint8_t* gq, const uint8_t* uq, const uint8_t* dq, int n,
                  int topk, int H, int I, int E, long grb, long urb, long drb, float* h_act,
                  float* dpart, float* out, int* dispatch, hipStream_t s) {
    GgMoeArgs a{gt, ut, dt, x, ids, w, gq, uq, dq, grb, urb, drb, n, topk, H, I, E, h_act, dpart,
                dispatch, nullptr, nullptr, nullptr, nullptr};
    return gg_moe<false>(a, out, dispatch, s);
}

int launch_gg_moe_i8(uint32_t gt, uint32_t ut, uint32_t dt, const int8_t* xq, const float* xs,
                     const int* ids, const float* w, const uint8_t* gq, const uint8_t* uq,
                     const uint8_t* dq, int n, int topk, int H, int I, int E, long grb, long urb,
                     long drb, float* h_act, int8_t* hq, float* hs, float* dpart, float* out,
                     int* dispatch, hipStream_t s) {
    GgMoeArgs a{gt, ut, dt, nullptr, ids, w, gq, uq, dq, grb, urb, drb, n, topk, H, I, E, h_act,
                dpart, dispatch, xq, xs, hq, hs};
    return gg_moe<true>(a, out, dispatch, s);
}

}  // namespace glmmoe
