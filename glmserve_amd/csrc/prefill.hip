// W4A16 experts, large-group regime (prefill and wide verify batches):
// grouped GEMM tiles of 128 grouped rows x 128 features (gate/up) or
// 256 features (down) on bf16 MFMA 32x32x16.
//
// Reference: the expert-major tensor-core path of the reference's GGUF MoE
// (cuda/qgemm.cu:1269-1356, emajor_mma_s8_kernel, used once n*topk reaches
// GLMSERVE_MMA_MOE_MIN_TS) and its W4A16 expert FFN semantics
// (cuda/moe_expert.cu:143-222).
//
// Workgroup = 8 waves as a 4 (features) x 2 (rows) grid; every wave owns 64
// features x 64 rows = 2 x 2 MFMA blocks of 32 x 32. For gate/up a wave's two
// feature blocks are 32 gate features and the same 32 up features, so
// SiLU(g) * u is formed in registers. The K loop runs over 128-K groups (one
// int4 scale group): per group, the workgroup's 16 weight tiles (16 KiB), their
// scales, the group sums of the 128 rows and the 128 activation rows
// (gathered by token id for gate/up) are streamed global -> LDS by LDS-DMA into
// a 3-slot ring, as in the decode kernels: each wave issues the same kDma DMAs
// per group, waits with an immediate vmcnt, and one s_barrier per group
// publishes the slot.
//
// Per group and 32 x 32 block: P = sum_k (128 + c) x over the group's 128 K
// (8 MFMAs), then acc += scale_row * (P - 136 * X_col), where X_col is the
// group sum of the column's activations: xsum from the router pass for gate/up,
// and for down the hsum this kernel's gate/up epilogue writes (the 4 feature
// waves of a workgroup cover exactly one 128-feature group of h).
//
// MFMA 32x32x16 is used because on gfx950 it sustains ~2.2 PFLOP/s of bf16
// where 16x16x32 reaches ~1.2 (measured with back-to-back independent chains).
#include "common.hpp"
#include "bigtile.hpp"
#include "kernels.hpp"

namespace glmmoe {

struct BigArgs {
    const uint4* wq[2];
    const uint16_t* ws[2];
    const uint4* swq[2];
    const uint16_t* sws[2];
    const uint16_t* src;     // x [n, H] (NMAT = 2, rows gathered) or h [R, I] (NMAT = 1)
    const float* gsum;       // xsum [n, H/128] (NMAT = 2) or hsum [R, I/128] (NMAT = 1)
    const int4* tiles; const int* ntiles; const int* rows_tok;
    uint16_t* h; float* hsum; float* dpart;
    int H, I, E;
};

constexpr int kBigD = 3;

struct BigRing {
    static constexpr int kWBytes = 16 * 1024;           // 16 weight tiles of 1 KiB
    static constexpr int kSOff = kWBytes;               // scales: tile t at 32 t (512 B)
    static constexpr int kGOff = kSOff + 512;           // group sums: row r at 4 r (512 B)
    static constexpr int kJunk = kGOff + 512;           // target of the placeholder DMAs
    static constexpr int kXOff = kJunk + 256;
    static constexpr int kQuad = 1024 + 64;             // one DMA = 4 rows x 256 B (+ pad)
    static constexpr int kSlot = kXOff + (kBigRows / 4) * kQuad;
    static constexpr int kBytes = kBigD * kSlot;
    static constexpr int kRed = kBytes;                 // [4][128] floats: h group-sum partials
    static constexpr int kTab = kRed + 4 * kBigRows * 4;
    static constexpr int kTotal = kTab + kBigTable * kBigTabInts * 4;
    static_assert(kTotal <= 160 * 1024, "one workgroup's LDS");
#ifdef GLMMOE_BIG_NODMA
    static constexpr int kDma = 0;   // diagnostics: compute on stale LDS, no streaming
#else
    static constexpr int kDma = 2 + 1 + 1 + 4;          // per wave per group
#endif
    // A DMA block holds 4 rows interleaved at 16 B: chunk c (8 bf16) of row r
    // sits at block(r / 4) + 64 c + 16 (r % 4); with the 1088-byte block stride
    // the 32 rows an MFMA fragment reads fall on distinct banks.
    static __device__ __forceinline__ int row_off(int r) { return (r >> 2) * kQuad + (r & 3) * 16; }
};

template <int NMAT>
struct BigShape {
    static constexpr int kFeat = NMAT == 2 ? 128 : 256;   // features per item
};

// Tile t (0..15) of an item: weight matrix and 16-row feature block. Tiles
// 4 wn .. 4 wn + 3 belong to feature wave wn: for gate/up, 2 gate tiles then
// the 2 up tiles of the same 32 features; for down, 4 consecutive tiles.
template <int NMAT>
__device__ __forceinline__ void tile_of(int t, int g, int& m, int& fb) {
    if (NMAT == 2) {
        m = (t & 3) >> 1;
        fb = g * 8 + (t >> 2) * 2 + (t & 1);
    } else {
        m = 0;
        fb = g * 16 + t;
    }
}

template <int NMAT>
__device__ __forceinline__ void big_issue(const BigArgs& a, const BigItem& it, int kg, int K,
                                          int KG, char* slot, int wave, int lane) {
    using RG = BigRing;
#ifdef GLMMOE_BIG_NODMA
    return;
#endif
    const bool sh = it.e == a.E;
    const int frows = NMAT == 2 ? a.I : a.H;
    const size_t mstride_q = (size_t)(frows / 16) * KG * 64;
    const size_t mstride_s = (size_t)(frows / 16) * KG * 16;
    const uint4* wbase[2];
    const uint16_t* sbase[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const int mm = m < NMAT ? m : 0;
        wbase[m] = sh ? a.swq[mm] : a.wq[mm] + (size_t)it.e * mstride_q;
        sbase[m] = sh ? a.sws[mm] : a.ws[mm] + (size_t)it.e * mstride_s;
    }
    // Weight tiles 2 wave, 2 wave + 1.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int t = wave * 2 + j;
        int m, fb;
        tile_of<NMAT>(t, it.g, m, fb);
        dma16(wbase[m] + ((size_t)fb * KG + kg) * 64 + lane, slot + t * 1024);
    }
    // Scales: waves 0 / 1 fetch tiles 0-7 / 8-15 (lane -> tile lane / 8, dword
    // lane % 8); the other waves issue a placeholder so every wave issues kDma.
    {
        const int t = (wave & 1) * 8 + (lane >> 3);
        int m, fb;
        tile_of<NMAT>(t, it.g, m, fb);
        dma4(sbase[m] + ((size_t)fb * KG + kg) * 16 + (lane & 7) * 2,
             slot + (wave < 2 ? RG::kSOff + (wave & 1) * 256 : RG::kJunk));
    }
    // Group sums: waves 2 / 3 fetch rows 0-63 / 64-127 (lane = row).
    {
        const int row = (wave & 1) * 64 + lane;
        const int rr = row < it.nr ? row : 0;
        const float* gp;
        if (NMAT == 2) {
            const uint32_t tok = lds_read32(it.tab + 16 + rr * 4);
            gp = a.gsum + (size_t)tok * KG + kg;
        } else {
            gp = a.gsum + (size_t)(it.r0 + rr) * KG + kg;
        }
        dma4(gp, slot + ((wave >> 1) == 1 ? RG::kGOff + (wave & 1) * 256 : RG::kJunk));
    }
    // Rows wave*16 .. wave*16+15: 4 DMAs of 4 rows x 256 B, rows interleaved
    // at 16 B (lane -> row lane % 4, chunk lane / 4).
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int sub = lane & 3;
        const int chunk = lane >> 2;
        const uint4 t4 = lds_bcast16(it.tab + 16 + (wave * 16 + j * 4) * 4);
        const uint32_t tk = sub == 0 ? t4.x : sub == 1 ? t4.y : sub == 2 ? t4.z : t4.w;
        dma16(a.src + (size_t)tk * K + kg * 128 + chunk * 8,
              slot + RG::kXOff + (wave * 4 + j) * RG::kQuad);
    }
}

// One 128-K group of the wave's 64 x 64 tile. Row blocks at or past nr
// (padding of an expert's last tile) are skipped; nr is wave-uniform.
__device__ __forceinline__ void big_compute(const char* slot, int wave, int lane, int nr,
                                            const DqConst& dqc, f32x16 (&acc)[2][2]) {
    using RG = BigRing;
    const int wn = wave >> 1, wm = wave & 1;
    const int col = lane & 31, h = lane >> 5;
    const int ntb = min(2, max(0, (nr - wm * 64 + 31) >> 5));   // live 32-row blocks
    if (ntb == 0) return;
    // A fragments: block jb = tiles 4 wn + 2 jb (+1 for rows 16-31); lane row
    // col holds K chunks 8h .. 8h+7 = packed-tile lane slots q = 2h, 2h+1.
    u32x4 aw[2][2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
        const int t = wn * 4 + jb * 2 + (col >> 4);
        const uint32_t wa = lds_addr(slot + t * 1024) + (uint32_t)(((col & 15) + 32 * h) * 16);
        asm volatile("ds_read_b128 %0, %2\n ds_read_b128 %1, %2 offset:256"
                     : "=&v"(aw[jb][0]), "=&v"(aw[jb][1]) : "v"(wa));
    }
    // Scales of this lane's 16 output rows per block: rows 8j + 4h + [0, 4).
    u32x2 sv[2][4];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = 8 * j + 4 * h;
            const int t = wn * 4 + jb * 2 + (row >> 4);
            const uint32_t sa = lds_addr(slot + RG::kSOff + t * 32) + (uint32_t)((row & 15) * 2);
            asm volatile("ds_read_b64 %0, %1" : "=&v"(sv[jb][j]) : "v"(sa));
        }
    // Group sums of this lane's two columns.
    float xs[2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        const uint32_t ga = lds_addr(slot + RG::kGOff) + (uint32_t)((wm * 64 + tb * 32 + col) * 4);
        asm volatile("ds_read_b32 %0, %1" : "=&v"(xs[tb]) : "v"(ga));
    }
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(aw[0][0]), "+v"(aw[0][1]), "+v"(aw[1][0]), "+v"(aw[1][1]),
                   "+v"(sv[0][0]), "+v"(sv[0][1]), "+v"(sv[0][2]), "+v"(sv[0][3]),
                   "+v"(sv[1][0]), "+v"(sv[1][1]), "+v"(sv[1][2]), "+v"(sv[1][3]),
                   "+v"(xs[0]), "+v"(xs[1]));
    const uint32_t xb = lds_addr(slot + RG::kXOff);
    uint32_t xa[2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
        xa[tb] = xb + (uint32_t)(RG::row_off(wm * 64 + tb * 32 + col) + 8 * h * 64);

    // Activation fragments double-buffered across the 8 K-steps: the reads of
    // step s+1 are in flight during step s's MFMAs.
    f32x16 p[2][2];
    u32x4 xv[2][2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
        asm volatile("ds_read_b128 %0, %1" : "=&v"(xv[0][tb]) : "v"(xa[tb]));
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const int cb = s & 1, nb = cb ^ 1;
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(xv[cb][0]), "+v"(xv[cb][1]));
        if (s < 7) {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
                asm volatile("ds_read_b128 %0, %1 offset:%c2"
                             : "=&v"(xv[nb][tb]) : "v"(xa[tb]), "i"((s + 1) * 64));
        }
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
            const bf16x8 av = dq_w4(aw[jb][s >> 2][s & 3], dqc);
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                if (tb < ntb) {
                    if (s == 0) p[jb][tb] = mfma32x32x16(av, as_bf16x8(xv[cb][tb]), f32x16{});
                    else p[jb][tb] = mfma32x32x16(av, as_bf16x8(xv[cb][tb]), p[jb][tb]);
                }
            }
        }
    }
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
        float sc[16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            sc[4 * j + 0] = bf16_to_f32(sv[jb][j].x & 0xffffu);
            sc[4 * j + 1] = bf16_to_f32(sv[jb][j].x >> 16);
            sc[4 * j + 2] = bf16_to_f32(sv[jb][j].y & 0xffffu);
            sc[4 * j + 3] = bf16_to_f32(sv[jb][j].y >> 16);
        }
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            if (tb < ntb) {
                const float off = -136.0f * xs[tb];
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    acc[jb][tb][i] = __builtin_fmaf(sc[i], p[jb][tb][i] + off, acc[jb][tb][i]);
            }
        }
    }
}

template <int NMAT>
__device__ __forceinline__ void big_epilogue(const BigArgs& a, const BigItem& cur, char* lds,
                                             int wave, int lane, f32x16 (&acc)[2][2]) {
    const int wn = wave >> 1, wm = wave & 1;
    const int col = lane & 31, h = lane >> 5;
    if constexpr (NMAT == 2) {
        // h = silu(g) * u (bf16) for 32 features x this lane's 2 columns; and
        // the sum of the rounded h over the workgroup's 128 features (one
        // group of I), reduced across the 4 feature waves in fixed order.
        float part[2];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            const int lr = wm * 64 + tb * 32 + col;
            const bool valid = lr < cur.nr;
            const size_t row = (size_t)cur.r0 + lr;
            float ps = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t hb[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    hb[e] = f32_to_bf16(silu_fast(acc[0][tb][4 * j + e]) * acc[1][tb][4 * j + e]);
                    ps += bf16_to_f32(hb[e]);
                }
                const int f = cur.g * 128 + wn * 32 + 8 * j + 4 * h;
                if (valid)
                    *reinterpret_cast<uint2*>(a.h + row * a.I + f) =
                        uint2{hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16)};
            }
            part[tb] = ps + __shfl_xor(ps, 32);   // both row halves of the 32 features
        }
        const uint32_t red = lds_addr(lds + BigRing::kRed);
        if (h == 0) {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
                lds_write32(red + (uint32_t)((wn * kBigRows + wm * 64 + tb * 32 + col) * 4), part[tb]);
        }
        __builtin_amdgcn_s_barrier();
        if (wn == 0 && h == 0) {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                const int lr = wm * 64 + tb * 32 + col;
                float s = 0.0f;
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    s += __uint_as_float(lds_read32(red + (uint32_t)((w * kBigRows + lr) * 4)));
                if (lr < cur.nr) a.hsum[((size_t)cur.r0 + lr) * (a.I / 128) + cur.g] = s;
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
__global__ __launch_bounds__(512) void w4_big_kernel(BigArgs a) {
    using RG = BigRing;
    extern __shared__ __align__(16) char lds[];
    const DqConst dqc = dq_const();
    int* table = reinterpret_cast<int*>(lds + RG::kTab);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = NMAT == 2 ? a.H : a.I;
    const int KG = K / 128;
    const int nfg = (NMAT == 2 ? a.I : a.H) / BigShape<NMAT>::kFeat;
    const long total = (long)(*a.ntiles) * nfg;
    const long nitems = big_rounds(total);

    for (long k0 = 0; k0 < nitems; k0 += kBigTable) {
        const int cnt = (int)min((long)kBigTable, nitems - k0);
        big_fill_table<NMAT == 2>(a.tiles, a.rows_tok, table, k0, cnt, nfg);
        __syncthreads();
        const long nsteps = (long)cnt * KG;

        int iss_k = 0, iss_g = 0;
        BigItem iss = big_item(lds + RG::kTab, 0);
        for (int j = 0; j < kBigD - 1; ++j) {
            if (j < nsteps) {
                big_issue<NMAT>(a, iss, iss_g, K, KG, lds + (j % kBigD) * RG::kSlot, wave, lane);
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
            if (step + kBigD - 2 < nsteps) wait_vmcnt<RG::kDma * (kBigD - 2)>();
            else wait_vmcnt<0>();
            __builtin_amdgcn_s_barrier();
            if (step + kBigD - 1 < nsteps) {
                big_issue<NMAT>(a, iss, iss_g, K, KG, lds + ((step + kBigD - 1) % kBigD) * RG::kSlot,
                                wave, lane);
                if (++iss_g == KG) {
                    iss_g = 0;
                    if (++iss_k < cnt) iss = big_item(lds + RG::kTab, iss_k);
                }
            }
#ifndef GLMMOE_BIG_NOCOMPUTE
            big_compute(lds + (step % kBigD) * RG::kSlot, wave, lane, cur.nr, dqc, acc);
#endif

            if (++cur_g == KG) {
                big_epilogue<NMAT>(a, cur, lds, wave, lane, acc);
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
static int launch_big(const BigArgs& a, long max_items, hipStream_t s) {
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&w4_big_kernel<NMAT>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, BigRing::kTotal) !=
            hipSuccess)
            return -4;
        attr_set = true;
    }
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    long blocks = max_items < cus ? max_items : cus;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL((w4_big_kernel<NMAT>), dim3((unsigned)blocks), dim3(512), BigRing::kTotal,
                       s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_gate_up_big(const ExpertPtrs& P, const uint16_t* x, const float* xsum,
                       const int* tiles, const int* ntiles, int max_tiles, const int* rows_tok,
                       uint16_t* h, float* hsum, int H, int I, int E, hipStream_t s) {
    BigArgs a{};
    a.wq[0] = reinterpret_cast<const uint4*>(P.gate_q); a.ws[0] = P.gate_s;
    a.wq[1] = reinterpret_cast<const uint4*>(P.up_q); a.ws[1] = P.up_s;
    a.swq[0] = reinterpret_cast<const uint4*>(P.sh_gate_q); a.sws[0] = P.sh_gate_s;
    a.swq[1] = reinterpret_cast<const uint4*>(P.sh_up_q); a.sws[1] = P.sh_up_s;
    a.src = x; a.gsum = xsum; a.tiles = reinterpret_cast<const int4*>(tiles); a.ntiles = ntiles;
    a.rows_tok = rows_tok; a.h = h; a.hsum = hsum; a.H = H; a.I = I; a.E = E;
    return launch_big<2>(a, (long)max_tiles * (I / BigShape<2>::kFeat), s);
}

int launch_down_big(const ExpertPtrs& P, const uint16_t* h, const float* hsum, const int* tiles,
                    const int* ntiles, int max_tiles, float* dpart, int H, int I, int E,
                    hipStream_t s) {
    BigArgs a{};
    a.wq[0] = reinterpret_cast<const uint4*>(P.down_q); a.ws[0] = P.down_s;
    a.swq[0] = reinterpret_cast<const uint4*>(P.sh_down_q); a.sws[0] = P.sh_down_s;
    a.wq[1] = a.wq[0]; a.ws[1] = a.ws[0]; a.swq[1] = a.swq[0]; a.sws[1] = a.sws[0];
    a.src = h; a.gsum = hsum; a.tiles = reinterpret_cast<const int4*>(tiles); a.ntiles = ntiles;
    a.dpart = dpart; a.H = H; a.I = I; a.E = E;
    return launch_big<1>(a, (long)max_tiles * (H / BigShape<1>::kFeat), s);
}

}  // namespace glmmoe
