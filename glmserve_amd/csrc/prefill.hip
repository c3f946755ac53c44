// W4A16 experts, large-group regime (prefill and wide verify batches):
// grouped GEMM tiles of 128 grouped rows x 128 features (gate/up) or
// 256 features (down) on bf16 MFMA.
//
// Reference: the expert-major tensor-core path of the reference's GGUF MoE
// (cuda/qgemm.cu:1269-1356, emajor_mma_s8_kernel, used once n*topk reaches
// GLMSERVE_MMA_MOE_MIN_TS) and its W4A16 expert FFN semantics
// (cuda/moe_expert.cu:143-222).
//
// Workgroup = 8 waves as a 4 (features) x 2 (rows) grid; every wave owns 64
// features x 64 rows = 4 x 4 MFMA blocks of 16 x 16. For gate/up a wave's 4
// feature blocks are 2 gate + the 2 matching up blocks, so SiLU(g) * u is
// formed in registers. The K loop runs over 128-K groups (one int4 scale
// group): per group, the workgroup's 16 weight tiles (16 KiB), scales and
// the 128 activation rows (gathered by token id for gate/up) are streamed
// global -> LDS by LDS-DMA into a 3-slot ring, exactly as in the decode
// kernels: each wave issues the same kDma DMAs per group, waits with an
// immediate vmcnt, and one s_barrier per group publishes the slot.
// Per group and 16 x 16 block: P = sum_k (128 + c) x over the group's 128 K
// (4 MFMAs), the group sum X_j from an all-ones MFMA, then
//   acc += scale_row * (P - 136 * X_j).
#include "common.hpp"
#include "kernels.hpp"

namespace glmmoe {

struct BigArgs {
    const uint4* wq[2];
    const uint16_t* ws[2];
    const uint4* swq[2];
    const uint16_t* sws[2];
    const uint16_t* src;     // x [n, H] (NMAT = 2, rows gathered) or h [R, I] (NMAT = 1)
    const int4* tiles; const int* ntiles; const int* rows_tok;
    uint16_t* h; float* dpart;
    int H, I, E;
};

constexpr int kBigWaves = 8;
constexpr int kBigD = 3;
constexpr int kBigTable = 8;              // items per table refill
constexpr int kBigTabInts = 4 + kBigRows; // {expert, row0, nrows, feature group} + tokens

template <int NMAT>
struct BigRing {
    static constexpr int kWBytes = 16 * 1024;           // 16 weight tiles of 1 KiB
    static constexpr int kSBytes = kBigWaves * 256;     // per-wave scale dwords
    static constexpr int kQuad = 1024 + 16;             // one DMA = 4 rows x 256 B (+ pad)
    static constexpr int kXBytes = (kBigRows / 4) * kQuad;
    static constexpr int kSlot = kWBytes + kSBytes + kXBytes;
    static constexpr int kBytes = kBigD * kSlot;
    static constexpr int kTotal = kBytes + kBigTable * kBigTabInts * 4;
    static constexpr int kDma = 2 + 1 + 4;              // per wave per group
    static constexpr int kFeat = NMAT == 2 ? 128 : 256; // features per item
    static __device__ __forceinline__ int row_off(int r) { return (r >> 2) * kQuad + (r & 3) * 256; }
};

struct BigItem {
    int e, r0, nr, g;
    uint32_t tab;              // LDS address of the item's table entry
};

__device__ __forceinline__ BigItem big_item(const int* table, int k) {
    const uint32_t base = lds_addr(table + k * kBigTabInts);
    const uint4 hd = lds_bcast16(base);
    BigItem it;
    it.e = sgpr(hd.x);
    it.r0 = sgpr(hd.y);
    it.nr = sgpr(hd.z);
    it.g = sgpr(hd.w);
    it.tab = base;
    return it;
}

// Tile t (0..15) of an item: the weight matrix and 16-row feature block.
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
    using RG = BigRing<NMAT>;
    const int wn = wave >> 1, wm = wave & 1;
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
    // This wave's 2 of the 16 weight tiles (the pair its row-partner also reads).
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int t = wn * 4 + wm * 2 + j;
        int m, fb;
        tile_of<NMAT>(t, it.g, m, fb);
        dma16(wbase[m] + ((size_t)fb * KG + kg) * 64 + lane, slot + t * 1024);
    }
    // Scales of the wave's own 4 tiles: lane l -> tile (l / 8) % 4, dword l % 8.
    {
        const int jj = (lane >> 3) & 3;
        int m, fb;
        tile_of<NMAT>(wn * 4 + jj, it.g, m, fb);
        dma4(sbase[m] + ((size_t)fb * KG + kg) * 16 + (lane & 7) * 2,
             slot + RG::kWBytes + wave * 256);
    }
    // Rows wave*16 .. wave*16+15: 4 DMAs of 4 rows x 256 B.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int sub = lane >> 4;
        const uint4 t4 = lds_bcast16(it.tab + 16 + (wave * 16 + j * 4) * 4);
        const uint32_t tk = sub == 0 ? t4.x : sub == 1 ? t4.y : sub == 2 ? t4.z : t4.w;
        const size_t srow = (size_t)tk;
        dma16(a.src + srow * K + kg * 128 + (lane & 15) * 8,
              slot + RG::kWBytes + RG::kSBytes + (wave * 4 + j) * RG::kQuad);
    }
}

template <int NMAT>
__device__ __forceinline__ void big_compute(const char* slot, int wave, int lane,
                                            f32x4 (&acc)[4][4]) {
    using RG = BigRing<NMAT>;
    const int wn = wave >> 1, wm = wave & 1;
    const int r = lane & 15, q = lane >> 4;
    const uint32_t xb = lds_addr(slot + RG::kWBytes + RG::kSBytes);
    uint4 xf[4][4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
        const uint32_t xa = xb + (uint32_t)(RG::row_off(wm * 64 + tb * 16 + r) + q * 64);
        asm volatile(
            "ds_read_b128 %0, %4\n"
            "ds_read_b128 %1, %4 offset:16\n"
            "ds_read_b128 %2, %4 offset:32\n"
            "ds_read_b128 %3, %4 offset:48\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(xf[tb][0]), "=&v"(xf[tb][1]), "=&v"(xf[tb][2]), "=&v"(xf[tb][3])
            : "v"(xa));
    }
    const bf16x8 ones = __builtin_bit_cast(bf16x8, uint4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
    float off[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
        f32x4 px = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int d = 0; d < 4; ++d) px = mfma16x16x32(ones, as_bf16x8(xf[tb][d]), px);
        off[tb] = -136.0f * px[0];
    }
    const uint32_t wa0 = lds_addr(slot) + (uint32_t)(wn * 4 * 1024 + lane * 16);
    const uint32_t sa0 = lds_addr(slot + RG::kWBytes + wave * 256) + (uint32_t)(q * 8);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint4 w;
        uint2 sv;
        asm volatile(
            "ds_read_b128 %0, %2\n"
            "ds_read_b64 %1, %3\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(w), "=&v"(sv)
            : "v"(wa0 + j * 1024), "v"(sa0 + j * 32));
        const float sc[4] = {bf16_to_f32(sv.x & 0xffffu), bf16_to_f32(sv.x >> 16),
                             bf16_to_f32(sv.y & 0xffffu), bf16_to_f32(sv.y >> 16)};
        const bf16x8 a0 = dq_w4(w.x), a1 = dq_w4(w.y), a2 = dq_w4(w.z), a3 = dq_w4(w.w);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            f32x4 p = {0.f, 0.f, 0.f, 0.f};
            p = mfma16x16x32(a0, as_bf16x8(xf[tb][0]), p);
            p = mfma16x16x32(a1, as_bf16x8(xf[tb][1]), p);
            p = mfma16x16x32(a2, as_bf16x8(xf[tb][2]), p);
            p = mfma16x16x32(a3, as_bf16x8(xf[tb][3]), p);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc[j][tb][e] = __builtin_fmaf(sc[e], p[e] + off[tb], acc[j][tb][e]);
        }
    }
}

template <int NMAT>
__device__ __forceinline__ void big_fill_table(const BigArgs& a, int* table, long k0, int cnt,
                                               int nfg) {
    for (int i = threadIdx.x; i < cnt * kBigTabInts; i += blockDim.x) {
        const int k = i / kBigTabInts, f = i % kBigTabInts;
        const long item = (long)blockIdx.x + (k0 + k) * gridDim.x;
        const int4 tile = a.tiles[item / nfg];
        int v;
        if (f == 0) v = tile.x;
        else if (f == 1) v = tile.y;
        else if (f == 2) v = tile.z;
        else if (f == 3) v = (int)(item % nfg);
        else {
            const int row = f - 4;
            const int rr = row < tile.z ? row : 0;
            v = NMAT == 2 ? a.rows_tok[tile.y + rr] : tile.y + rr;
        }
        table[i] = v;
    }
}

template <int NMAT>
__global__ __launch_bounds__(512) void w4_big_kernel(BigArgs a) {
    using RG = BigRing<NMAT>;
    extern __shared__ __align__(16) char ring[];
    int* table = reinterpret_cast<int*>(ring + RG::kBytes);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wn = wave >> 1, wm = wave & 1;
    const int r = lane & 15, q = lane >> 4;
    const int K = NMAT == 2 ? a.H : a.I;
    const int KG = K / 128;
    const int nfg = (NMAT == 2 ? a.I : a.H) / RG::kFeat;
    const long total = (long)(*a.ntiles) * nfg;
    const long nitems = (long)blockIdx.x < total ? (total - blockIdx.x + gridDim.x - 1) / gridDim.x : 0;

    for (long k0 = 0; k0 < nitems; k0 += kBigTable) {
        const int cnt = (int)min((long)kBigTable, nitems - k0);
        big_fill_table<NMAT>(a, table, k0, cnt, nfg);
        __syncthreads();
        const long nsteps = (long)cnt * KG;

        int iss_k = 0, iss_g = 0;
        BigItem iss = big_item(table, 0);
        for (int j = 0; j < kBigD - 1; ++j) {
            if (j < nsteps) {
                big_issue<NMAT>(a, iss, iss_g, K, KG, ring + (j % kBigD) * RG::kSlot, wave, lane);
                if (++iss_g == KG) {
                    iss_g = 0;
                    if (++iss_k < cnt) iss = big_item(table, iss_k);
                }
            }
        }
        int cur_k = 0, cur_g = 0;
        BigItem cur = big_item(table, 0);
        f32x4 acc[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) acc[j][tb] = f32x4{0.f, 0.f, 0.f, 0.f};

        for (long step = 0; step < nsteps; ++step) {
            if (step + kBigD - 2 < nsteps) wait_vmcnt<RG::kDma * (kBigD - 2)>();
            else wait_vmcnt<0>();
            __builtin_amdgcn_s_barrier();
            if (step + kBigD - 1 < nsteps) {
                big_issue<NMAT>(a, iss, iss_g, K, KG,
                                ring + ((step + kBigD - 1) % kBigD) * RG::kSlot, wave, lane);
                if (++iss_g == KG) {
                    iss_g = 0;
                    if (++iss_k < cnt) iss = big_item(table, iss_k);
                }
            }
            big_compute<NMAT>(ring + (step % kBigD) * RG::kSlot, wave, lane, acc);

            if (++cur_g == KG) {
#pragma unroll
                for (int tb = 0; tb < 4; ++tb) {
                    const int lr = wm * 64 + tb * 16 + r;     // row inside the tile
                    const bool valid = lr < cur.nr;
                    const size_t row = (size_t)cur.r0 + lr;
                    if constexpr (NMAT == 2) {
#pragma unroll
                        for (int jj = 0; jj < 2; ++jj) {
                            uint32_t hb[4];
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                hb[e] = f32_to_bf16(silu_fast(acc[jj][tb][e]) * acc[2 + jj][tb][e]);
                            const int f = cur.g * 128 + wn * 32 + jj * 16 + 4 * q;
                            if (valid)
                                *reinterpret_cast<uint2*>(a.h + row * a.I + f) =
                                    uint2{hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16)};
                        }
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const int f = cur.g * 256 + wn * 64 + j * 16 + 4 * q;
                            if (valid)
                                *reinterpret_cast<float4*>(a.dpart + row * a.H + f) =
                                    make_float4(acc[j][tb][0], acc[j][tb][1], acc[j][tb][2],
                                                acc[j][tb][3]);
                        }
                    }
                }
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int tb = 0; tb < 4; ++tb) acc[j][tb] = f32x4{0.f, 0.f, 0.f, 0.f};
                cur_g = 0;
                if (++cur_k < cnt) cur = big_item(table, cur_k);
            }
        }
        __syncthreads();
    }
}

template <int NMAT>
static int launch_big(const BigArgs& a, long max_items, hipStream_t s) {
    using RG = BigRing<NMAT>;
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&w4_big_kernel<NMAT>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, RG::kTotal) !=
            hipSuccess)
            return -4;
        attr_set = true;
    }
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    long blocks = max_items < cus ? max_items : cus;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL((w4_big_kernel<NMAT>), dim3((unsigned)blocks), dim3(512), RG::kTotal, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_gate_up_big(const ExpertPtrs& P, const uint16_t* x, const int* tiles,
                       const int* ntiles, int max_tiles, const int* rows_tok, uint16_t* h, int H,
                       int I, int E, hipStream_t s) {
    BigArgs a{};
    a.wq[0] = reinterpret_cast<const uint4*>(P.gate_q); a.ws[0] = P.gate_s;
    a.wq[1] = reinterpret_cast<const uint4*>(P.up_q); a.ws[1] = P.up_s;
    a.swq[0] = reinterpret_cast<const uint4*>(P.sh_gate_q); a.sws[0] = P.sh_gate_s;
    a.swq[1] = reinterpret_cast<const uint4*>(P.sh_up_q); a.sws[1] = P.sh_up_s;
    a.src = x; a.tiles = reinterpret_cast<const int4*>(tiles); a.ntiles = ntiles;
    a.rows_tok = rows_tok; a.h = h; a.H = H; a.I = I; a.E = E;
    return launch_big<2>(a, (long)max_tiles * (I / BigRing<2>::kFeat), s);
}

int launch_down_big(const ExpertPtrs& P, const uint16_t* h, const int* tiles, const int* ntiles,
                    int max_tiles, float* dpart, int H, int I, int E, hipStream_t s) {
    BigArgs a{};
    a.wq[0] = reinterpret_cast<const uint4*>(P.down_q); a.ws[0] = P.down_s;
    a.swq[0] = reinterpret_cast<const uint4*>(P.sh_down_q); a.sws[0] = P.sh_down_s;
    a.wq[1] = a.wq[0]; a.ws[1] = a.ws[0]; a.swq[1] = a.swq[0]; a.sws[1] = a.sws[0];
    a.src = h; a.tiles = reinterpret_cast<const int4*>(tiles); a.ntiles = ntiles;
    a.dpart = dpart; a.H = H; a.I = I; a.E = E;
    return launch_big<1>(a, (long)max_tiles * (H / BigRing<1>::kFeat), s);
}

}  // namespace glmmoe
