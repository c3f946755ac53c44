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
    // Activation rows are 128 B, row r at 128 r, so one DMA (64 lanes x 16 B)
    // reads 8 whole rows with adjacent lanes on adjacent bytes (full-speed L2
    // coalescing). Chunk c of row r sits at slot c ^ ((r >> 1) & 7): the 16
    // rows an MFMA fragment pass reads at one chunk land on 16 distinct bank
    // groups.
    static constexpr int kSOff = kXOff + kBigRows * 128;          // activation scales
    static constexpr int kWSOff = kSOff + 4 * kBigRows;          // weight block scales
    static constexpr int kJunk = kWSOff + 256;                   // placeholder DMA target
    static constexpr int kSlot = kJunk + 256;
    static constexpr int kBytes = kF8D * kSlot;
    static constexpr int kRed = kBytes;                          // [4][128] floats
    static constexpr int kTab = kRed + 4 * kBigRows * 4;
    static constexpr int kTotal = kTab + kBigTable * kBigTabInts * 4;
    static_assert(kTotal <= 160 * 1024, "one workgroup's LDS");
    static constexpr int kDma = 4 + 2 + 1;                       // per wave per group
    static __device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }
};

// DMA sources of one item at K-group 0 (group kg adds kg * 4 KiB to the weight
// stream, kg * 128 B to the activation rows and kg to the scale streams).
struct F8Issue {
    const uint8_t* w;        // this wave's weight tile (lane offset included)
    const float* sc;         // wave 0: weight block scale; waves 1, 2: activation scale
    uint32_t x[2];           // src offsets of this lane's 16 B in the two activation DMAs
};

template <int NMAT>
__device__ __forceinline__ F8Issue f8_issue_ptrs(const F8Args& a, const BigItem& it, int K, int KG,
                                                 int wave, int lane) {
    F8Issue p;
    const bool sh = it.e == a.E;
    const int frows = NMAT == 2 ? a.I : a.H;
    const size_t mstride_q = (size_t)frows * K;
    const size_t mstride_s = (size_t)(frows / 128) * KG;
    {
        // Weight tile of this wave: (wn, jb) = (wave / 2, wave % 2).
        const int wn = wave >> 1, jb = wave & 1;
        const int m = NMAT == 2 ? jb : 0;
        const int fb = NMAT == 2 ? it.g * 4 + wn : it.g * 8 + wn * 2 + jb;
        const uint8_t* base = sh ? a.swq[m] : a.wq[m] + (size_t)it.e * mstride_q;
        p.w = base + (size_t)fb * KG * 4096 + lane * 16;
    }
    // Activation DMA j of this wave fills rows 8 (2 wave + j) + lane / 8; the
    // lane's LDS slot lane % 8 holds chunk (lane % 8) ^ swz(row).
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int row = (wave * 2 + j) * 8 + (lane >> 3);
        const uint32_t tk = lds_read32(it.tab + 16 + row * 4);
        p.x[j] = tk * (uint32_t)K + (uint32_t)(((lane & 7) ^ F8Ring::swz(row)) * 16);
    }
    // Scales: wave 0 the weight block scales (lane & 1 -> gate / up, or the
    // down item's two 128-feature blocks); waves 1 / 2 the activation scales
    // of rows 0-63 / 64-127; other waves a placeholder.
    if (wave == 0) {
        const float* sb0 = sh ? a.sws[0] : a.ws[0] + (size_t)it.e * mstride_s;
        const float* sb1 = sh ? a.sws[1] : a.ws[1] + (size_t)it.e * mstride_s;
        const bool odd = lane & 1;
        const float* sb = NMAT == 2 && odd ? sb1 : sb0;
        const int fblk = NMAT == 2 ? it.g : it.g * 2 + (odd ? 1 : 0);
        p.sc = sb + (size_t)fblk * KG;
    } else if (wave == 1 || wave == 2) {
        const int row = (wave - 1) * 64 + lane;
        const uint32_t tk = lds_read32(it.tab + 16 + row * 4);
        p.sc = a.sscale + (size_t)tk * KG;
    } else {
        p.sc = a.sscale;
    }
    return p;
}

// Exactly kDma DMAs per wave: group kg of the item into `slot`.
__device__ __forceinline__ void f8_issue(const F8Args& a, const F8Issue& p, int kg, char* slot,
                                         int wave) {
    using RG = F8Ring;
    const uint8_t* src = p.w + (size_t)kg * 4096;
    char* dst = slot + wave * 4096;
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(src + j * 1024, dst + j * 1024);
#pragma unroll
    for (int j = 0; j < 2; ++j)
        dma16(a.src + (p.x[j] + (uint32_t)kg * 128), slot + RG::kXOff + (wave * 2 + j) * 1024);
    char* sdst = wave == 0 ? slot + RG::kWSOff
               : (wave == 1 || wave == 2) ? slot + RG::kSOff + (wave - 1) * 256
               : slot + RG::kJunk;
    dma4(wave < 3 ? p.sc + kg : p.sc, sdst);
}

// Operands a wave reads from one ring slot for one 64-K half (K step s) of a
// group: chunk rows 2 s, 2 s + 1 of its two weight blocks and, of its two
// 32-row activation blocks, chunks 4 s + 2 h + {0, 1} (K step s, half h,
// 16-B piece q at chunk 4 s + 2 h + q). Row R = wm * 64 + tb * 32 + col
// (tb = 1 is 32 rows = 4 KiB further, same swizzle); chunk c at slot
// c ^ swz(R).
struct F8Half {
    u32x4 aw[2][2];
    u32x4 bx[2][2];
};

template <int S>
__device__ __forceinline__ void f8_load_half(const char* slot, int wave, int lane, F8Half& o) {
    using RG = F8Ring;
    const int wn = wave >> 1, wm = wave & 1;
    const int col = lane & 31, h = lane >> 5;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
        const uint32_t wa = lds_addr(slot + (wn * 2 + jb) * 4096) + (uint32_t)(lane * 16);
        asm volatile("ds_read_b128 %0, %2 offset:%3\n ds_read_b128 %1, %2 offset:%4"
                     : "=&v"(o.aw[jb][0]), "=&v"(o.aw[jb][1])
                     : "v"(wa), "n"(2048 * S), "n"(2048 * S + 1024));
    }
    const int R = wm * 64 + col;
    const uint32_t xr = lds_addr(slot + RG::kXOff) + (uint32_t)(R * 128);
    const int f = RG::swz(R);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t xa = xr + (uint32_t)((((4 * S + 2 * h + q) ^ f)) * 16);
        asm volatile("ds_read_b128 %0, %2\n ds_read_b128 %1, %2 offset:4096"
                     : "=&v"(o.bx[0][q]), "=&v"(o.bx[1][q]) : "v"(xa));
    }
}

// The activation scales of the wave's rows and the weight block scales.
__device__ __forceinline__ void f8_load_scales(const char* slot, int wave, int lane, int nmat, float (&xs)[2],
                                               float (&ws)[2]) {
    using RG = F8Ring;
    const int wn = wave >> 1, wm = wave & 1;
    const int R = wm * 64 + (lane & 31);
    const uint32_t sa = lds_addr(slot + RG::kSOff) + (uint32_t)(R * 4);
    asm volatile("ds_read_b32 %0, %2\n ds_read_b32 %1, %2 offset:128" : "=&v"(xs[0]), "=&v"(xs[1]) : "v"(sa));
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
        const int idx = nmat == 2 ? jb : (wn >> 1);
        const uint32_t wa = lds_addr(slot + RG::kWSOff) + (uint32_t)(idx * 4);
        asm volatile("ds_read_b32 %0, %1" : "=&v"(ws[jb]) : "v"(wa));
    }
}

__device__ __forceinline__ void f8_wait_half(F8Half& o) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(o.aw[0][0]), "+v"(o.aw[0][1]), "+v"(o.aw[1][0]), "+v"(o.aw[1][1]),
                   "+v"(o.bx[0][0]), "+v"(o.bx[0][1]), "+v"(o.bx[1][0]), "+v"(o.bx[1][1]));
}
__device__ __forceinline__ void f8_wait_half(F8Half& o, float (&xs)[2], float (&ws)[2]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(o.aw[0][0]), "+v"(o.aw[0][1]), "+v"(o.aw[1][0]), "+v"(o.aw[1][1]),
                   "+v"(o.bx[0][0]), "+v"(o.bx[0][1]), "+v"(o.bx[1][0]), "+v"(o.bx[1][1]),
                   "+v"(xs[0]), "+v"(xs[1]), "+v"(ws[0]), "+v"(ws[1]));
}

// K step S of a group: p = A . B over the half's 64 K (S = 0 from zero).
template <int S>
__device__ __forceinline__ void f8_mfma_half(const F8Half& o, f32x16 (&p)[2][2]) {
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
            p[jb][tb] = mfma_f8_32x32x64(cat8(o.aw[jb][0], o.aw[jb][1]), cat8(o.bx[tb][0], o.bx[tb][1]),
                                         S == 0 ? f32x16{} : p[jb][tb]);
}

// acc += (w_scale * x_scale) * p.
__device__ __forceinline__ void f8_rescale(const float (&xs)[2], const float (&ws)[2],
                                           const f32x16 (&p)[2][2], f32x16 (&acc)[2][2]) {
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            const float sc = ws[jb] * xs[tb];
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[jb][tb][i] = __builtin_fmaf(sc, p[jb][tb][i], acc[jb][tb][i]);
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
                        // bf16 partial rows (the combine adds them in fp32).
                        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.dpart) + row * a.H + f) =
                            uint2{pack_bf16x2(acc[jb][tb][4 * j], acc[jb][tb][4 * j + 1]),
                                  pack_bf16x2(acc[jb][tb][4 * j + 2], acc[jb][tb][4 * j + 3])};
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
    const int wm = wave & 1;
    const int K = NMAT == 2 ? a.H : a.I;
    const int KG = K / 128;
    const int nfg = NMAT == 2 ? a.I / 128 : a.H / 256;
    const int nitems = (int)big_rounds((long)(*a.ntiles) * nfg);

    for (int k0 = 0; k0 < nitems; k0 += kBigTable) {
        const int cnt = min(kBigTable, nitems - k0);
        big_fill_table_em<NMAT == 2>(a.tiles, a.rows_tok, table, k0, cnt, nfg);
        __syncthreads();
        const int nsteps = cnt * KG;

        // Ring of kF8D slots, group g in slot g % kF8D. Per group: compute g;
        // wait for g + 1's DMA and barrier (every wave is then done with slot
        // g, and g + 1 is visible); refill slot g with group g + kF8D; issue
        // the reads of g + 1's operands; apply g's scales under those reads.
        int iss_k = 0, iss_g = 0;
        F8Issue iss = f8_issue_ptrs<NMAT>(a, big_item(lds + RG::kTab, 0), K, KG, wave, lane);
        auto issue_next = [&](int g) {
            f8_issue(a, iss, iss_g, lds + (g % kF8D) * RG::kSlot, wave);
            if (++iss_g == KG) {
                iss_g = 0;
                if (++iss_k < cnt)
                    iss = f8_issue_ptrs<NMAT>(a, big_item(lds + RG::kTab, iss_k), K, KG, wave, lane);
            }
        };
        for (int j = 0; j < kF8D; ++j)
            if (j < nsteps) issue_next(j);
        if (nsteps >= 3) wait_vmcnt<RG::kDma * 2>();
        else if (nsteps == 2) wait_vmcnt<RG::kDma>();
        else wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        // Operands by 64-K half: h0 (K step 0) of the current group, h1 (K
        // step 1); its scales in xs / ws, the next group's in nxs / nws.
        F8Half h0, h1;
        float xs[2], ws[2], nxs[2], nws[2];
        f8_load_half<0>(lds, wave, lane, h0);
        f8_load_scales(lds, wave, lane, NMAT, xs, ws);
        f8_wait_half(h0, xs, ws);

        int cur_k = 0, cur_g = 0;
        BigItem cur = big_item(lds + RG::kTab, 0);
        // Whether this wave's 64 rows hold any live row (wave-uniform per item).
        bool live = cur.nr > wm * 64;
        f32x16 acc[2][2];
#pragma unroll
        for (int jb = 0; jb < 2; ++jb)
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) acc[jb][tb] = f32x16{};

        for (int step = 0; step < nsteps; ++step) {
            // Half 1's reads go out under half 0's MFMAs; after the barrier
            // the next group's half 0 (and scales) under half 1's MFMAs and
            // this group's rescale. Every wave has its reads of slot g in
            // (waited before the barrier) when slot g is refilled.
            const char* slot = lds + (step % kF8D) * RG::kSlot;
            f32x16 p[2][2];
            f8_load_half<1>(slot, wave, lane, h1);
            if (live) f8_mfma_half<0>(h0, p);
            f8_wait_half(h1);
            if (step + 2 < nsteps) wait_vmcnt<RG::kDma>();
            else wait_vmcnt<0>();
            __builtin_amdgcn_s_barrier();
            if (step + kF8D < nsteps) issue_next(step + kF8D);
            if (step + 1 < nsteps) {
                const char* nslot = lds + ((step + 1) % kF8D) * RG::kSlot;
                f8_load_half<0>(nslot, wave, lane, h0);
                f8_load_scales(nslot, wave, lane, NMAT, nxs, nws);
            }
            if (live) {
                f8_mfma_half<1>(h1, p);
                f8_rescale(xs, ws, p, acc);
            }
            if (++cur_g == KG) {
                f8_epilogue<NMAT>(a, cur, lds, wave, lane, acc);
#pragma unroll
                for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                    for (int tb = 0; tb < 2; ++tb) acc[jb][tb] = f32x16{};
                cur_g = 0;
                if (++cur_k < cnt) {
                    cur = big_item(lds + RG::kTab, cur_k);
                    live = cur.nr > wm * 64;
                }
            }
            // Last in the iteration: the next group's operands have arrived
            // before anything (including copies the compiler makes for the
            // loop) reads their registers.
            f8_wait_half(h0, nxs, nws);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                xs[i] = nxs[i];
                ws[i] = nws[i];
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
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
