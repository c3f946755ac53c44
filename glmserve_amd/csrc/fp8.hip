// FP8 (e4m3, OCP "fn" encoding) experts: block-scaled weights, per-token
// per-128-channel activations, gfx950 fp8 MFMA.
//
// Format. Weights: e4m3 bytes [rows, K] with one fp32 scale per 128 x 128
// block ([rows/128, K/128]), w = e4m3(q) * scale (the block-scaled FP8
// checkpoint layout; the reference's FP8 code decodes e4m3 with a per-row
// scale only, cuda/fp8_gemm.cu:14-35, include/common.hpp:182-200).
// Activations: per token and 128 channels, scale = amax / 448 (1 for an all
// zero group), q = e4m3(x / scale), round-to-nearest-even, saturating to
// +-448 so the NaN codes 0x7f / 0xff never appear. The SwiGLU intermediate h
// is quantized by the same rule inside the gate/up epilogue.
//
// Kernels:
//   quant_act_kernel  bf16 -> e4m3 + scales (x before the gate/up GEMM).
//   pack_fp8_kernel   row-major e4m3 -> MFMA-native 32-row x 128-K tiles.
//   fp8_big_kernel    grouped GEMM over 128-row tiles, same work decomposition
//                     and LDS-DMA ring as the W4A16 large-group kernel; per
//                     128-K group and 32 x 32 block two MFMA 32x32x64 fp8
//                     products P, then acc += (w_scale * x_scale) * P.
#include "bigtile.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace glmmoe {

typedef int i32x8 __attribute__((ext_vector_type(8)));

// D = A . B over 64 K of e4m3 (cbsz = blgp = 0: both operands e4m3), the
// block-scale operands at 127 (E8M0 for 2^0). Lane l of A holds row l % 32,
// of B column l % 32; both hold the same 32 K positions, so any fixed
// lane -> K assignment shared by the two operands gives the same product.
__device__ __forceinline__ f32x16 mfma_f8_32x32x64(i32x8 a, i32x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

__device__ __forceinline__ i32x8 cat8(u32x4 lo, u32x4 hi) {
    return __builtin_bit_cast(i32x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// f32 -> e4m3 code, round-to-nearest-even, saturating at 448 (NaN -> 448 with
// its sign bit). Normal range: keep 3 mantissa bits of the f32 pattern with
// RNE by integer add (a carry into the exponent is the correct rounding);
// subnormal range (< 2^-6): the value in units of 2^-9, rounded by rint.
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
    const uint32_t sign = (__float_as_uint(f) >> 24) & 0x80u;
    const float a = __builtin_fabsf(f);
    uint32_t code;
    if (!(a < 448.0f)) {
        code = 0x7eu;
    } else if (a < 0.015625f) {
        code = (uint32_t)__builtin_rintf(a * 512.0f);
    } else {
        uint32_t b = __float_as_uint(a);
        b += 0x7ffffu + ((b >> 20) & 1u);
        code = (b >> 20) - (120u << 3);
    }
    return sign | code;
}

// Quantization scale of a group with maximum magnitude amax.
__device__ __forceinline__ float e4m3_group_scale(float amax) {
    return amax > 0.0f ? __fdiv_rn(amax, 448.0f) : 1.0f;
}

// ---------------------------------------------------------------------------
// x bf16 [n, K] -> q e4m3 [n, K], scale fp32 [n, K/128]. 16 lanes per group,
// 8 channels (16 B) per lane.
__global__ __launch_bounds__(256) void quant_act_kernel(const uint16_t* __restrict__ x,
                                                        long ngroups, uint8_t* __restrict__ q,
                                                        float* __restrict__ scale) {
    const long gi = ((long)blockIdx.x * 256 + threadIdx.x) >> 4;
    const int sub = threadIdx.x & 15;
    const bool ok = gi < ngroups;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (ok) v = reinterpret_cast<const uint4*>(x + gi * 128)[sub];
    float f[8];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = bf16_to_f32(w[i] & 0xffffu);
        f[2 * i + 1] = bf16_to_f32(w[i] >> 16);
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, __builtin_fabsf(f[i]));
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 16));
    const float s = e4m3_group_scale(amax);
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        lo |= f32_to_e4m3(__fdiv_rn(f[i], s)) << (8 * i);
        hi |= f32_to_e4m3(__fdiv_rn(f[4 + i], s)) << (8 * i);
    }
    if (ok) {
        reinterpret_cast<uint2*>(q + gi * 128)[sub] = make_uint2(lo, hi);
        if (sub == 0) scale[gi] = s;
    }
}

int launch_quant_act_fp8(const uint16_t* x, int n, int K, uint8_t* q, float* scale,
                         hipStream_t s) {
    const long ngroups = (long)n * (K / 128);
    const long blocks = (ngroups * 16 + 255) / 256;
    hipLaunchKernelGGL(quant_act_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, ngroups, q,
                       scale);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// ---------------------------------------------------------------------------
// Native weight tiles: [mat][32-row block fb][128-K group kg][4 KiB]. In a tile,
// 16-byte chunk (j, lane) (j = 0..3, lane = 0..63) holds row fb * 32 + lane % 32,
// K = kg * 128 + 64 (j / 2) + 32 (lane / 32) + 16 (j % 2) + [0, 16): one
// ds_read_b128 of chunk row j by the 64 lanes is half of an MFMA A operand
// (K step j / 2), and one LDS-DMA of 1 KiB moves a chunk row.
__global__ __launch_bounds__(256) void pack_fp8_kernel(const uint4* __restrict__ w, long nchunks,
                                                       int rows, int K,
                                                       uint4* __restrict__ out) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= nchunks) return;
    const int KG = K / 128;
    const int lane = (int)(i & 63);
    const int j = (int)((i >> 6) & 3);
    const long tile = i >> 8;
    const int kg = (int)(tile % KG);
    const long mfb = tile / KG;                      // mat * (rows / 32) + fb
    const long row = mfb * 32 + (lane & 31);         // row within all matrices
    const int k = kg * 128 + 64 * (j >> 1) + 32 * (lane >> 5) + 16 * (j & 1);
    out[i] = w[(row * K + k) / 16];
}

int launch_pack_fp8(const uint8_t* w, int n_mats, int rows, int K, uint8_t* packed,
                    hipStream_t s) {
    const long nchunks = (long)n_mats * rows * K / 16;
    hipLaunchKernelGGL(pack_fp8_kernel, dim3((unsigned)((nchunks + 255) / 256)), dim3(256), 0, s,
                       reinterpret_cast<const uint4*>(w), nchunks, rows, K,
                       reinterpret_cast<uint4*>(packed));
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// ---------------------------------------------------------------------------
// Grouped GEMM over 128-row tiles.
//
// Workgroup = 8 waves as 4 (features) x 2 (rows); every wave owns 64 features x
// 64 rows = 2 x 2 blocks of 32 x 32. Gate/up items cover 128 features of h:
// wave wn's block 0 is gate rows g*128 + 32 wn + [0, 32), block 1 the same up
// rows. Down items cover 256 output features: wave wn's blocks are 32-row
// blocks 8 g + 2 wn + {0, 1}. Per 128-K group the workgroup streams 8 weight
// tiles (32 KiB), its 128 activation rows (16 KiB), their scales and the
// weight block scales into a 3-slot LDS ring by LDS-DMA (7 DMAs per wave).
struct F8Args {
    const uint8_t* wq[2];
    const float* ws[2];
    const uint8_t* swq[2];
    const float* sws[2];
    const uint8_t* src;      // xq [n, H] (gate/up, rows gathered) or hq [R, I] (down)
    const float* sscale;     // its scales [.., K/128]
    const int4* tiles; const int* ntiles; const int* rows_tok;
    uint8_t* hq; float* hscale; float* dpart;
    int H, I, E;
};

constexpr int kF8D = 3;

struct F8Ring {
    static constexpr int kWBytes = 8 * 4096;            // 8 weight tiles
    static constexpr int kXOff = kWBytes;
    // One activation DMA = 8 rows x 128 B, chunk c of row r at 128 c + 16 (r % 8);
    // the 1152-byte block stride puts rows 8..15 of a 16-lane read phase on
    // the other half of the banks.
    static constexpr int kOct = 1024 + 128;
    static constexpr int kSOff = kXOff + (kBigRows / 8) * kOct;   // activation scales
    static constexpr int kWSOff = kSOff + 4 * kBigRows;          // weight block scales
    static constexpr int kJunk = kWSOff + 256;                   // placeholder DMA target
    static constexpr int kSlot = kJunk + 256;
    static constexpr int kBytes = kF8D * kSlot;
    static constexpr int kRed = kBytes;                          // [4][128] floats
    static constexpr int kTab = kRed + 4 * kBigRows * 4;
    static constexpr int kTotal = kTab + kBigTable * kBigTabInts * 4;
    static_assert(kTotal <= 160 * 1024, "one workgroup's LDS");
    static constexpr int kDma = 4 + 2 + 1;                       // per wave per group
    static __device__ __forceinline__ int row_off(int r) { return (r >> 3) * kOct + (r & 7) * 16; }
};

template <int NMAT>
__device__ __forceinline__ void f8_issue(const F8Args& a, const BigItem& it, int kg, int K, int KG,
                                         char* slot, int wave, int lane) {
    using RG = F8Ring;
    const bool sh = it.e == a.E;
    const int frows = NMAT == 2 ? a.I : a.H;
    const size_t mstride_q = (size_t)frows * K;
    const size_t mstride_s = (size_t)(frows / 128) * KG;
    // Weight tile of this wave: (wn, jb) = (wave / 2, wave % 2).
    {
        const int wn = wave >> 1, jb = wave & 1;
        const int m = NMAT == 2 ? jb : 0;
        const int fb = NMAT == 2 ? it.g * 4 + wn : it.g * 8 + wn * 2 + jb;
        const uint8_t* base = sh ? a.swq[m] : a.wq[m] + (size_t)it.e * mstride_q;
        const uint8_t* src = base + ((size_t)fb * KG + kg) * 4096 + lane * 16;
        char* dst = slot + wave * 4096;
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16(src + j * 1024, dst + j * 1024);
    }
    // Activation rows 16 wave .. 16 wave + 15: lane -> row lane % 8, chunk lane / 8.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int blk = wave * 2 + j;
        const int row = blk * 8 + (lane & 7);
        const uint32_t tk = lds_read32(it.tab + 16 + row * 4);
        dma16(a.src + (size_t)tk * K + kg * 128 + (lane >> 3) * 16,
              slot + RG::kXOff + blk * RG::kOct);
    }
    // Scales: wave 0 the weight block scales (lane & 1 -> gate / up, or the
    // down item's two 128-feature blocks); waves 1 / 2 the activation scales
    // of rows 0-63 / 64-127; other waves a placeholder.
    if (wave == 0) {
        // Both candidate bases are wave-uniform; the per-lane choice is a
        // select (indexing the argument array by lane would load it from memory).
        const float* sb0 = sh ? a.sws[0] : a.ws[0] + (size_t)it.e * mstride_s;
        const float* sb1 = sh ? a.sws[1] : a.ws[1] + (size_t)it.e * mstride_s;
        const bool odd = lane & 1;
        const float* sb = NMAT == 2 && odd ? sb1 : sb0;
        const int fblk = NMAT == 2 ? it.g : it.g * 2 + (odd ? 1 : 0);
        dma4(sb + (size_t)fblk * KG + kg, slot + RG::kWSOff);
    } else if (wave == 1 || wave == 2) {
        const int row = (wave - 1) * 64 + lane;
        const uint32_t tk = lds_read32(it.tab + 16 + row * 4);
        dma4(a.sscale + (size_t)tk * KG + kg, slot + RG::kSOff + (wave - 1) * 256);
    } else {
        dma4(a.sscale, slot + RG::kJunk);
    }
}

template <int NMAT>
__device__ __forceinline__ void f8_compute(const char* slot, int wave, int lane, int nr,
                                           f32x16 (&acc)[2][2]) {
    using RG = F8Ring;
    const int wn = wave >> 1, wm = wave & 1;
    const int col = lane & 31, h = lane >> 5;
    const int ntb = min(2, max(0, (nr - wm * 64 + 31) >> 5));   // live 32-row blocks
    if (ntb == 0) return;
    u32x4 aw[2][4];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
        const uint32_t wa = lds_addr(slot + (wn * 2 + jb) * 4096) + (uint32_t)(lane * 16);
        asm volatile(
            "ds_read_b128 %0, %4\n ds_read_b128 %1, %4 offset:1024\n"
            " ds_read_b128 %2, %4 offset:2048\n ds_read_b128 %3, %4 offset:3072"
            : "=&v"(aw[jb][0]), "=&v"(aw[jb][1]), "=&v"(aw[jb][2]), "=&v"(aw[jb][3])
            : "v"(wa));
    }
    // B: row r's K chunk 4 s + 2 h + q, matching A's chunk (j = 2 s + q, half h).
    u32x4 bx[2][4];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        const int row = wm * 64 + tb * 32 + col;
        const uint32_t xa =
            lds_addr(slot + RG::kXOff) + (uint32_t)(RG::row_off(row) + 2 * h * 128);
        asm volatile(
            "ds_read_b128 %0, %4\n ds_read_b128 %1, %4 offset:128\n"
            " ds_read_b128 %2, %4 offset:512\n ds_read_b128 %3, %4 offset:640"
            : "=&v"(bx[tb][0]), "=&v"(bx[tb][1]), "=&v"(bx[tb][2]), "=&v"(bx[tb][3])
            : "v"(xa));
    }
    float xs[2], ws[2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        const uint32_t sa = lds_addr(slot + RG::kSOff) + (uint32_t)((wm * 64 + tb * 32 + col) * 4);
        asm volatile("ds_read_b32 %0, %1" : "=&v"(xs[tb]) : "v"(sa));
    }
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
        const int idx = NMAT == 2 ? jb : (wn >> 1);
        const uint32_t wa = lds_addr(slot + RG::kWSOff) + (uint32_t)(idx * 4);
        asm volatile("ds_read_b32 %0, %1" : "=&v"(ws[jb]) : "v"(wa));
    }
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(aw[0][0]), "+v"(aw[0][1]), "+v"(aw[0][2]), "+v"(aw[0][3]),
                   "+v"(aw[1][0]), "+v"(aw[1][1]), "+v"(aw[1][2]), "+v"(aw[1][3]),
                   "+v"(bx[0][0]), "+v"(bx[0][1]), "+v"(bx[0][2]), "+v"(bx[0][3]),
                   "+v"(bx[1][0]), "+v"(bx[1][1]), "+v"(bx[1][2]), "+v"(bx[1][3]),
                   "+v"(xs[0]), "+v"(xs[1]), "+v"(ws[0]), "+v"(ws[1]));
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            if (tb < ntb) {
                f32x16 p = mfma_f8_32x32x64(cat8(aw[jb][0], aw[jb][1]),
                                            cat8(bx[tb][0], bx[tb][1]), f32x16{});
                p = mfma_f8_32x32x64(cat8(aw[jb][2], aw[jb][3]), cat8(bx[tb][2], bx[tb][3]), p);
                const float sc = ws[jb] * xs[tb];
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[jb][tb][i] = __builtin_fmaf(sc, p[i], acc[jb][tb][i]);
            }
        }
    }
}

template <int NMAT>
__device__ __forceinline__ void f8_epilogue(const F8Args& a, const BigItem& cur, char* lds,
                                            int wave, int lane, f32x16 (&acc)[2][2]) {
    const int wn = wave >> 1, wm = wave & 1;
    const int col = lane & 31, h = lane >> 5;
    if constexpr (NMAT == 2) {
        // h = silu(g) * u for 32 features x this lane's 2 rows; amax over the
        // item's 128 features (one quantization group of h) via LDS, then e4m3.
        float hv[2][16], part[2];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            float m = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                hv[tb][i] = silu_fast(acc[0][tb][i]) * acc[1][tb][i];
                m = fmaxf(m, __builtin_fabsf(hv[tb][i]));
            }
            part[tb] = fmaxf(m, __shfl_xor(m, 32));
        }
        const uint32_t red = lds_addr(lds + F8Ring::kRed);
        if (h == 0) {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
                lds_write32(red + (uint32_t)((wn * kBigRows + wm * 64 + tb * 32 + col) * 4), part[tb]);
        }
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            const int lr = wm * 64 + tb * 32 + col;
            float amax = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w)
                amax = fmaxf(amax, __uint_as_float(lds_read32(red + (uint32_t)((w * kBigRows + lr) * 4))));
            const float s = e4m3_group_scale(amax);
            if (lr < cur.nr) {
                const size_t row = (size_t)cur.r0 + lr;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uint32_t word = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        word |= f32_to_e4m3(__fdiv_rn(hv[tb][4 * j + e], s)) << (8 * e);
                    const int f = cur.g * 128 + wn * 32 + 8 * j + 4 * h;
                    *reinterpret_cast<uint32_t*>(a.hq + row * a.I + f) = word;
                }
                if (wn == 0 && h == 0) a.hscale[row * (a.I / 128) + cur.g] = s;
            }
        }
        __builtin_amdgcn_s_barrier();   // partials consumed before the next item reuses them
    } else {
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            const int lr = wm * 64 + tb * 32 + col;
            if (lr < cur.nr) {
                const size_t row = (size_t)cur.r0 + lr;
#pragma unroll
                for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int f = cur.g * 256 + wn * 64 + jb * 32 + 8 * j + 4 * h;
                        *reinterpret_cast<float4*>(a.dpart + row * a.H + f) =
                            make_float4(acc[jb][tb][4 * j], acc[jb][tb][4 * j + 1],
                                        acc[jb][tb][4 * j + 2], acc[jb][tb][4 * j + 3]);
                    }
            }
        }
    }
}

template <int NMAT>
__global__ __launch_bounds__(512) void fp8_big_kernel(F8Args a) {
    using RG = F8Ring;
    extern __shared__ __align__(16) char lds[];
    int* table = reinterpret_cast<int*>(lds + RG::kTab);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = NMAT == 2 ? a.H : a.I;
    const int KG = K / 128;
    const int nfg = NMAT == 2 ? a.I / 128 : a.H / 256;
    const long nitems = big_rounds((long)(*a.ntiles) * nfg);

    for (long k0 = 0; k0 < nitems; k0 += kBigTable) {
        const int cnt = (int)min((long)kBigTable, nitems - k0);
        big_fill_table<NMAT == 2>(a.tiles, a.rows_tok, table, k0, cnt, nfg);
        __syncthreads();
        const long nsteps = (long)cnt * KG;

        int iss_k = 0, iss_g = 0;
        BigItem iss = big_item(lds + RG::kTab, 0);
        for (int j = 0; j < kF8D - 1; ++j) {
            if (j < nsteps) {
                f8_issue<NMAT>(a, iss, iss_g, K, KG, lds + (j % kF8D) * RG::kSlot, wave, lane);
                if (++iss_g == KG) {
                    iss_g = 0;
                    if (++iss_k < cnt) iss = big_item(lds + RG::kTab, iss_k);
                }
            }
        }
        int cur_k = 0, cur_g = 0;
        BigItem cur = big_item(lds + RG::kTab, 0);
        f32x16 acc[2][2];
#pragma unroll
        for (int jb = 0; jb < 2; ++jb)
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) acc[jb][tb] = f32x16{};

        for (long step = 0; step < nsteps; ++step) {
            if (step + kF8D - 2 < nsteps) wait_vmcnt<RG::kDma * (kF8D - 2)>();
            else wait_vmcnt<0>();
            __builtin_amdgcn_s_barrier();
            if (step + kF8D - 1 < nsteps) {
                f8_issue<NMAT>(a, iss, iss_g, K, KG, lds + ((step + kF8D - 1) % kF8D) * RG::kSlot,
                               wave, lane);
                if (++iss_g == KG) {
                    iss_g = 0;
                    if (++iss_k < cnt) iss = big_item(lds + RG::kTab, iss_k);
                }
            }
            f8_compute<NMAT>(lds + (step % kF8D) * RG::kSlot, wave, lane, cur.nr, acc);

            if (++cur_g == KG) {
                f8_epilogue<NMAT>(a, cur, lds, wave, lane, acc);
#pragma unroll
                for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                    for (int tb = 0; tb < 2; ++tb) acc[jb][tb] = f32x16{};
                cur_g = 0;
                if (++cur_k < cnt) cur = big_item(lds + RG::kTab, cur_k);
            }
        }
        __syncthreads();
    }
}

template <int NMAT>
static int launch_f8(const F8Args& a, long max_items, hipStream_t s) {
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&fp8_big_kernel<NMAT>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, F8Ring::kTotal) !=
            hipSuccess)
            return -4;
        attr_set = true;
    }
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    long blocks = max_items < cus ? max_items : cus;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL((fp8_big_kernel<NMAT>), dim3((unsigned)blocks), dim3(512), F8Ring::kTotal,
                       s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_gate_up_fp8(const Fp8Ptrs& P, const uint8_t* xq, const float* xscale,
                       const int* tiles, const int* ntiles, int max_tiles, const int* rows_tok,
                       uint8_t* hq, float* hscale, int H, int I, int E, hipStream_t s) {
    F8Args a{};
    a.wq[0] = P.gate_q; a.ws[0] = P.gate_s; a.wq[1] = P.up_q; a.ws[1] = P.up_s;
    a.swq[0] = P.sh_gate_q; a.sws[0] = P.sh_gate_s; a.swq[1] = P.sh_up_q; a.sws[1] = P.sh_up_s;
    a.src = xq; a.sscale = xscale; a.tiles = reinterpret_cast<const int4*>(tiles);
    a.ntiles = ntiles; a.rows_tok = rows_tok; a.hq = hq; a.hscale = hscale;
    a.H = H; a.I = I; a.E = E;
    return launch_f8<2>(a, (long)max_tiles * (I / 128), s);
}

int launch_down_fp8(const Fp8Ptrs& P, const uint8_t* hq, const float* hscale, const int* tiles,
                    const int* ntiles, int max_tiles, float* dpart, int H, int I, int E,
                    hipStream_t s) {
    F8Args a{};
    a.wq[0] = a.wq[1] = P.down_q; a.ws[0] = a.ws[1] = P.down_s;
    a.swq[0] = a.swq[1] = P.sh_down_q; a.sws[0] = a.sws[1] = P.sh_down_s;
    a.src = hq; a.sscale = hscale; a.tiles = reinterpret_cast<const int4*>(tiles);
    a.ntiles = ntiles; a.dpart = dpart; a.H = H; a.I = I; a.E = E;
    return launch_f8<1>(a, (long)max_tiles * (H / 256), s);
}

}  // namespace glmmoe
