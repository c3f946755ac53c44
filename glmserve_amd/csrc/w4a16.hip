// W4A16 experts: native weight packing, grouped gate/up/SiLU and down
// products on bf16 MFMA (v_mfma_f32_16x16x32_bf16), and the deterministic
// combine with the shared expert.
//
// Reference: cuda/moe_expert.cu:132-244 (moe_expert_w4_fused_kernel: one
// block per token, weights re-read per token), the shared expert chain of
// src/model_gpu.cpp:1486-1494, and the slot-order combine of
// cuda/qgemm.cu:943-955 / src/model_glm52.cpp:1133-1152.
//
// Work decomposition. The dispatch kernel lists "tiles": runs of at most
// kTileRows grouped rows of one expert (the shared expert is expert E, with
// one row per token). A work item is (tile, 16-row weight block); one wave
// runs one work item at a time, streaming that weight block's 1 KiB K-tiles
// once and applying each to every 16-token block of the tile, so each expert
// weight byte is read from HBM once per tile. The MFMA sees weights as the A
// operand (16 output features) and tokens as the B operand (16 tokens).
#include "common.hpp"
#include "kernels.hpp"

namespace glmmoe {

// ---------------------------------------------------------------------------
// Packing: reference layout [rows, K/2] u8 + scales [rows, K/128] -> native.
// One thread per output dword.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_w4_kernel(const uint8_t* __restrict__ q,
                                                      const void* __restrict__ sc,
                                                      int sc_bf16, long n_dw, int rows, int K,
                                                      uint32_t* __restrict__ pq,
                                                      uint16_t* __restrict__ ps) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_dw) return;
    const int KG = K / 128;
    const long per_mat = (long)rows / 16 * KG * 256;  // dwords per matrix
    const long mat = i / per_mat;
    long rem = i % per_mat;
    const int d = (int)(rem & 3);
    const int lane = (int)((rem >> 2) & 63);
    const long tile = rem >> 8;
    const int kg = (int)(tile % KG);
    const int rb = (int)(tile / KG);
    const int r = rb * 16 + (lane & 15);
    const int qq = lane >> 4;
    const int k0 = kg * 128 + 32 * qq + 8 * d;
    const uint8_t* src = q + ((size_t)mat * rows + r) * (K / 2) + k0 / 2;
    uint32_t out = 0;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint32_t b = src[s];
        out |= (b & 0xfu) << (4 * s);          // position 2s   -> nibble s
        out |= (b >> 4) << (4 * s + 16);       // position 2s+1 -> nibble s+4
    }
    pq[i] = out;
    if (d == 0 && qq == 0) {
        // Scale of (row r, group kg) -> packed [mat][rb][kg][16].
        const size_t si = ((size_t)mat * rows + r) * KG + kg;
        uint16_t v;
        if (sc_bf16) v = reinterpret_cast<const uint16_t*>(sc)[si];
        else v = (uint16_t)f32_to_bf16(reinterpret_cast<const float*>(sc)[si]);
        ps[(((size_t)mat * (rows / 16) + rb) * KG + kg) * 16 + (lane & 15)] = v;
    }
}

int launch_pack_w4(const uint8_t* q, const void* sc, int sc_bf16, int n_mats, int rows, int K,
                   uint8_t* pq, uint16_t* ps, hipStream_t s) {
    const long n_dw = (long)n_mats * rows * K / 8;
    hipLaunchKernelGGL(pack_w4_kernel, dim3((unsigned)((n_dw + 255) / 256)), dim3(256), 0, s,
                       q, sc, sc_bf16, n_dw, rows, K, reinterpret_cast<uint32_t*>(pq), ps);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// ---------------------------------------------------------------------------
// Grouped gate/up + SiLU.
// Lane l: r = l & 15 is both the weight row (A operand) and the token column
// (B operand / output column); q = l >> 4 selects the 32-K quarter of each
// 128-K tile. MFMA step d (0..3) covers K = 32q + 8d + [0,8) for this lane.
// Output lane layout: rows 4q + j (j = 0..3), column r.
// ---------------------------------------------------------------------------
struct GuArgs {
    const uint4* gq; const uint4* uq; const uint16_t* gs; const uint16_t* us;
    const uint4* sgq; const uint4* suq; const uint16_t* sgs; const uint16_t* sus;
    const uint16_t* x; const float* xsum;
    const int4* tiles; const int* ntiles; const int* rows_tok;
    uint16_t* h; float* hsum;
    int H, I, E;
};

template <int NB>
__global__ __launch_bounds__(256) void w4_gate_up_kernel(GuArgs a) {
    const int lane = threadIdx.x & 63;
    const int r = lane & 15, q = lane >> 4;
    const int KG = a.H / 128;
    const int nfb = a.I / 16;
    const long total = (long)(*a.ntiles) * nfb;
    const long nwaves = (long)gridDim.x * 4;
    for (long w = (long)blockIdx.x * 4 + (threadIdx.x >> 6); w < total; w += nwaves) {
        const int4 tile = a.tiles[w / nfb];
        const int fb = (int)(w % nfb);
        const int e = tile.x, r0 = tile.y, nr = tile.z;
        const bool sh = e == a.E;
        const size_t mstride_q = (size_t)nfb * KG * 64;   // uint4 per matrix
        const size_t mstride_s = (size_t)nfb * KG * 16;   // u16 per matrix
        const uint4* gq = (sh ? a.sgq : a.gq + (size_t)e * mstride_q) + (size_t)fb * KG * 64;
        const uint4* uq = (sh ? a.suq : a.uq + (size_t)e * mstride_q) + (size_t)fb * KG * 64;
        const uint16_t* gs = (sh ? a.sgs : a.gs + (size_t)e * mstride_s) + (size_t)fb * KG * 16;
        const uint16_t* us = (sh ? a.sus : a.us + (size_t)e * mstride_s) + (size_t)fb * KG * 16;
        const int nb = (nr + 15) >> 4;

        const uint16_t* xrow[NB];
        const float* xsr[NB];
        bool valid[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            valid[b] = b * 16 + r < nr;
            const int tok = valid[b] ? a.rows_tok[r0 + b * 16 + r] : 0;
            xrow[b] = a.x + (size_t)tok * a.H + 32 * q;
            xsr[b] = a.xsum + (size_t)tok * KG;
        }
        f32x4 accg[NB], accu[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            accg[b] = f32x4{0.f, 0.f, 0.f, 0.f};
            accu[b] = f32x4{0.f, 0.f, 0.f, 0.f};
        }

        for (int kg = 0; kg < KG; ++kg) {
            const uint4 wg = gq[(size_t)kg * 64 + lane];
            const uint4 wu = uq[(size_t)kg * 64 + lane];
            const uint2 sgv = *reinterpret_cast<const uint2*>(gs + (size_t)kg * 16 + 4 * q);
            const uint2 suv = *reinterpret_cast<const uint2*>(us + (size_t)kg * 16 + 4 * q);
            const float sg[4] = {bf16_to_f32(sgv.x & 0xffffu), bf16_to_f32(sgv.x >> 16),
                                 bf16_to_f32(sgv.y & 0xffffu), bf16_to_f32(sgv.y >> 16)};
            const float su[4] = {bf16_to_f32(suv.x & 0xffffu), bf16_to_f32(suv.x >> 16),
                                 bf16_to_f32(suv.y & 0xffffu), bf16_to_f32(suv.y >> 16)};
            const bf16x8 ag0 = dq_w4(wg.x), ag1 = dq_w4(wg.y), ag2 = dq_w4(wg.z), ag3 = dq_w4(wg.w);
            const bf16x8 au0 = dq_w4(wu.x), au1 = dq_w4(wu.y), au2 = dq_w4(wu.z), au3 = dq_w4(wu.w);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (b >= nb) break;
                uint4 x0 = {0, 0, 0, 0}, x1 = x0, x2 = x0, x3 = x0;
                float X = 0.0f;
                if (valid[b]) {
                    const uint4* xp = reinterpret_cast<const uint4*>(xrow[b] + kg * 128);
                    x0 = xp[0]; x1 = xp[1]; x2 = xp[2]; x3 = xp[3];
                    X = xsr[b][kg];
                }
                f32x4 pg = {0.f, 0.f, 0.f, 0.f}, pu = pg;
                pg = mfma16x16x32(ag0, as_bf16x8(x0), pg);
                pu = mfma16x16x32(au0, as_bf16x8(x0), pu);
                pg = mfma16x16x32(ag1, as_bf16x8(x1), pg);
                pu = mfma16x16x32(au1, as_bf16x8(x1), pu);
                pg = mfma16x16x32(ag2, as_bf16x8(x2), pg);
                pu = mfma16x16x32(au2, as_bf16x8(x2), pu);
                pg = mfma16x16x32(ag3, as_bf16x8(x3), pg);
                pu = mfma16x16x32(au3, as_bf16x8(x3), pu);
                const float off = -136.0f * X;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    accg[b][j] = __builtin_fmaf(sg[j], pg[j] + off, accg[b][j]);
                    accu[b][j] = __builtin_fmaf(su[j], pu[j] + off, accu[b][j]);
                }
            }
        }

        // Epilogue: h = silu(g) * u as bf16; partial group sums of the
        // rounded h over this block's 16 features.
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (b >= nb) break;
            uint32_t hb[4];
            float part = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float hv = silu_fast(accg[b][j]) * accu[b][j];
                hb[j] = f32_to_bf16(hv);
                part += bf16_to_f32(hb[j]);
            }
            part += __shfl_xor(part, 16);
            part += __shfl_xor(part, 32);
            if (valid[b]) {
                const size_t row = (size_t)r0 + b * 16 + r;
                uint2 st = {hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16)};
                *reinterpret_cast<uint2*>(a.h + row * a.I + fb * 16 + 4 * q) = st;
                if (q == 0) a.hsum[row * nfb + fb] = part;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Grouped down projection: dpart[row, :] = down_e . h[row, :] (unweighted).
// ---------------------------------------------------------------------------
struct DownArgs {
    const uint4* dq; const uint16_t* ds; const uint4* sdq; const uint16_t* sds;
    const uint16_t* h; const float* hsum;
    const int4* tiles; const int* ntiles;
    float* dpart;
    int H, I, E;
};

template <int NB>
__global__ __launch_bounds__(256) void w4_down_kernel(DownArgs a) {
    const int lane = threadIdx.x & 63;
    const int r = lane & 15, q = lane >> 4;
    const int KG = a.I / 128;
    const int nfb = a.H / 16;
    const int nhs = a.I / 16;   // h partial sums per row
    const long total = (long)(*a.ntiles) * nfb;
    const long nwaves = (long)gridDim.x * 4;
    for (long w = (long)blockIdx.x * 4 + (threadIdx.x >> 6); w < total; w += nwaves) {
        const int4 tile = a.tiles[w / nfb];
        const int fb = (int)(w % nfb);
        const int e = tile.x, r0 = tile.y, nr = tile.z;
        const bool sh = e == a.E;
        const size_t mstride_q = (size_t)nfb * KG * 64;
        const size_t mstride_s = (size_t)nfb * KG * 16;
        const uint4* dq = (sh ? a.sdq : a.dq + (size_t)e * mstride_q) + (size_t)fb * KG * 64;
        const uint16_t* ds = (sh ? a.sds : a.ds + (size_t)e * mstride_s) + (size_t)fb * KG * 16;
        const int nb = (nr + 15) >> 4;
        bool valid[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) valid[b] = b * 16 + r < nr;
        f32x4 acc[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};

        for (int kg = 0; kg < KG; ++kg) {
            const uint4 wd = dq[(size_t)kg * 64 + lane];
            const uint2 sv = *reinterpret_cast<const uint2*>(ds + (size_t)kg * 16 + 4 * q);
            const float sd[4] = {bf16_to_f32(sv.x & 0xffffu), bf16_to_f32(sv.x >> 16),
                                 bf16_to_f32(sv.y & 0xffffu), bf16_to_f32(sv.y >> 16)};
            const bf16x8 a0 = dq_w4(wd.x), a1 = dq_w4(wd.y), a2 = dq_w4(wd.z), a3 = dq_w4(wd.w);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (b >= nb) break;
                uint4 x0 = {0, 0, 0, 0}, x1 = x0, x2 = x0, x3 = x0;
                float X = 0.0f;
                if (valid[b]) {
                    const size_t row = (size_t)r0 + b * 16 + r;
                    const uint4* hp =
                        reinterpret_cast<const uint4*>(a.h + row * a.I + kg * 128 + 32 * q);
                    x0 = hp[0]; x1 = hp[1]; x2 = hp[2]; x3 = hp[3];
                    const float4* hs = reinterpret_cast<const float4*>(a.hsum + row * nhs + kg * 8);
                    const float4 s0 = hs[0], s1 = hs[1];
                    X = ((s0.x + s0.y) + (s0.z + s0.w)) + ((s1.x + s1.y) + (s1.z + s1.w));
                }
                f32x4 p = {0.f, 0.f, 0.f, 0.f};
                p = mfma16x16x32(a0, as_bf16x8(x0), p);
                p = mfma16x16x32(a1, as_bf16x8(x1), p);
                p = mfma16x16x32(a2, as_bf16x8(x2), p);
                p = mfma16x16x32(a3, as_bf16x8(x3), p);
                const float off = -136.0f * X;
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[b][j] = __builtin_fmaf(sd[j], p[j] + off, acc[b][j]);
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (b >= nb) break;
            if (valid[b]) {
                const size_t row = (size_t)r0 + b * 16 + r;
                *reinterpret_cast<float4*>(a.dpart + row * a.H + fb * 16 + 4 * q) =
                    make_float4(acc[b][0], acc[b][1], acc[b][2], acc[b][3]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Combine: out[t] = (((0 + w0*y0) + w1*y1) + ...) + y_shared, slot order then
// shared (src/model_glm52.cpp:1133-1152). Gather, no atomics: deterministic.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ dpart,
                                                      const int* __restrict__ inv,
                                                      const float* __restrict__ w, int n,
                                                      int topk, int H, int with_shared,
                                                      float* __restrict__ out) {
    const int t = blockIdx.y;
    const int f4 = blockIdx.x * blockDim.x + threadIdx.x;
    if (f4 * 4 >= H) return;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < topk; ++s) {
        const float ws = w[(size_t)t * topk + s];
        const float4 y = reinterpret_cast<const float4*>(dpart + (size_t)inv[(size_t)t * topk + s] * H)[f4];
        acc.x = acc.x + ws * y.x; acc.y = acc.y + ws * y.y;
        acc.z = acc.z + ws * y.z; acc.w = acc.w + ws * y.w;
    }
    if (with_shared) {
        const float4 y = reinterpret_cast<const float4*>(dpart + ((size_t)n * topk + t) * H)[f4];
        acc.x = acc.x + y.x; acc.y = acc.y + y.y; acc.z = acc.z + y.z; acc.w = acc.w + y.w;
    }
    reinterpret_cast<float4*>(out + (size_t)t * H)[f4] = acc;
}

// ---------------------------------------------------------------------------
static int grid_for(long max_work) {
    long blocks = (max_work + 3) / 4;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    return (int)blocks;
}

int launch_gate_up(const ExpertPtrs& P, const uint16_t* x, const float* xsum, const int* tiles,
                   const int* ntiles, int max_tiles, const int* rows_tok, uint16_t* h,
                   float* hsum, int H, int I, int E, hipStream_t s) {
    GuArgs a;
    a.gq = reinterpret_cast<const uint4*>(P.gate_q); a.uq = reinterpret_cast<const uint4*>(P.up_q);
    a.gs = P.gate_s; a.us = P.up_s;
    a.sgq = reinterpret_cast<const uint4*>(P.sh_gate_q); a.suq = reinterpret_cast<const uint4*>(P.sh_up_q);
    a.sgs = P.sh_gate_s; a.sus = P.sh_up_s;
    a.x = x; a.xsum = xsum; a.tiles = reinterpret_cast<const int4*>(tiles); a.ntiles = ntiles;
    a.rows_tok = rows_tok; a.h = h; a.hsum = hsum; a.H = H; a.I = I; a.E = E;
    hipLaunchKernelGGL(w4_gate_up_kernel<kTileRows / 16>, dim3(grid_for((long)max_tiles * (I / 16))),
                       dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_down(const ExpertPtrs& P, const uint16_t* h, const float* hsum, const int* tiles,
                const int* ntiles, int max_tiles, float* dpart, int H, int I, int E,
                hipStream_t s) {
    DownArgs a;
    a.dq = reinterpret_cast<const uint4*>(P.down_q); a.ds = P.down_s;
    a.sdq = reinterpret_cast<const uint4*>(P.sh_down_q); a.sds = P.sh_down_s;
    a.h = h; a.hsum = hsum; a.tiles = reinterpret_cast<const int4*>(tiles); a.ntiles = ntiles;
    a.dpart = dpart; a.H = H; a.I = I; a.E = E;
    hipLaunchKernelGGL(w4_down_kernel<kTileRows / 16>, dim3(grid_for((long)max_tiles * (H / 16))),
                       dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_combine(const float* dpart, const int* inv, const float* w, int n, int topk, int H,
                   int with_shared, float* out, hipStream_t s) {
    dim3 grid((unsigned)((H / 4 + 255) / 256), (unsigned)n);
    hipLaunchKernelGGL(combine_kernel, grid, dim3(256), 0, s, dpart, inv, w, n, topk, H,
                       with_shared, out);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace glmmoe
