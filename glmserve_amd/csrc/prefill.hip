// W4A16 experts, large-group regime (prefill and wide verify batches):
// grouped GEMM tiles of 128 grouped rows x 128 features (gate/up) or
// 256 features (down) on bf16 MFMA 32x32x16.
//
// Reference: the expert-major tensor-core path of the reference's GGUF MoE
// (cuda/qgemm.cu:1269-1356, emajor_mma_s8_kernel, used once n*topk reaches
// GLMSERVE_MMA_MOE_MIN_TS) and its W4A16 expert FFN semantics
// (cuda/moe_expert.cu:143-222).
//
// Workgroup = 8 waves as a 4 (features) x 2 (rows) grid; every wave owns
// 64 rows x 64 weight rows = 2 x 2 MFMA blocks of 32 x 32. The activations
// are the MFMA A operand (rows = grouped token rows) and the int4 weights the
// B operand (columns = output features), so each lane's output column is one
// feature and needs one weight scale per 128-K group. For gate/up a wave's two
// weight blocks are 32 gate features and the same 32 up features, so
// SiLU(g) * u is formed in registers.
//
// Streaming. The K loop runs over 128-K groups (one int4 scale group): per
// group, the workgroup's 16 weight tiles (16 KiB), their scales, the group
// sums of the 128 rows and the 128 activation rows (gathered by token id for
// gate/up) are copied global -> LDS by LDS-DMA into a 3-slot ring. Each wave
// issues the same kDma DMAs per group from per-lane source pointers computed
// once per work item, waits with an immediate vmcnt, and one s_barrier per
// group publishes the slot.
//
// Arithmetic per group and 32 x 32 block. The int4 code c decodes exactly to
// the bf16 of 128 + c (see dq_w4), so the MFMAs produce
//   P = sum_k (128 + c) x = sum_k (c - 8) x + 136 X,   X = sum_k x (group sum).
// The chain is seeded with -136 X from one extra MFMA whose A operand holds X
// split into bf16 hi + lo parts (K slots 0 and 1; X - hi is exact in fp32 and
// its bf16 rounding leaves a relative error below 2^-16 of X) against a
// constant B of -136; the seed depends only on the rows, so both weight
// blocks of a wave share it. Then acc += scale_col * P: one fma per
// accumulator element per group. X is xsum from the router pass for gate/up
// and, for down, the hsum this kernel's gate/up epilogue writes (the 4
// feature waves of a workgroup cover exactly one 128-feature group of h).
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
    uint16_t* h; float* hsum;
    float* dpart;            // NMAT = 1: bf16 [R, H] partial rows (in the fp32-sized region)
    int H, I, E;
};

constexpr int kBigD = 3;

// Two item shapes share the ring and the per-group DMA count. A 128-row item
// (8 waves as 4 features x 2 rows) covers 128 rows x 16 weight tiles; a
// 64-row item (an expert's last tile of at most 64 rows, 8 waves x 1 row
// block) covers 64 rows x 32 weight tiles, twice the features. Per group both
// move 48 KiB: 16 KiB of weights + 32 KiB of activation rows, or 32 + 16.
struct BigRing {
    // Slot: weight tile t at 1 KiB t; activation row r at kX128 + 256 r
    // (128-row item) or kX64 + 256 r (64-row item); scales of tile t at
    // kSOff + 32 t; row group sums at kGOff + 4 r.
    static constexpr int kX128 = 16 * 1024;
    static constexpr int kX64 = 32 * 1024;
    static constexpr int kSOff = 48 * 1024;             // 32 tiles x 32 B
    static constexpr int kGOff = kSOff + 1024;          // 128 rows x 4 B
    static constexpr int kQuad = 1024;                  // one DMA = 4 rows x 256 B
    static constexpr int kSlot = kGOff + 512;
    static constexpr int kBytes = kBigD * kSlot;
    static constexpr int kRed = kBytes;                 // [4][128] or [8][64] floats: h group-sum partials
    static constexpr int kTab = kRed + 4 * kBigRows * 4;
    static constexpr int kTotal = kTab + kBigTable * kBigTabInts * 4;
    static_assert(kTotal <= 160 * 1024, "one workgroup's LDS");
    static constexpr int kDma = 6;   // weight / activation DMAs per wave per group
    // Plus one small DMA in waves 0-2: the scales of all the item's tiles
    // (wave 0, 16 B per lane) and the row group sums (waves 1, 2: rows 0-63,
    // 64-127). Every DMA instruction holds a slot of the CU's memory queue,
    // so there are no placeholder DMAs to even the counts out; the waits
    // count per wave.
    // Activation rows are 256 B each, so one DMA of 64 lanes reads 4 whole
    // rows, 16 consecutive lanes per row (lanes that share cache lines are
    // adjacent, which the address coalescer needs for full L2 bandwidth).
    // Inside a row, 16-byte chunk c sits at slot c ^ (r & 15): the 16 rows an
    // MFMA fragment pass reads at one chunk land on 16 distinct bank groups.
    static __device__ __forceinline__ int row_off(int r) { return r * 256; }
};

template <int NMAT>
struct BigShape {
    static constexpr int kFeat = NMAT == 2 ? 128 : 256;   // features per 128-row item
};

// Wave geometry of an item: feature block wn, row half wm, activation area.
struct BigGeo {
    int wn, wm, xoff;
};
__device__ __forceinline__ BigGeo big_geo(int hs, int wave) {
    return hs ? BigGeo{wave, 0, BigRing::kX64} : BigGeo{wave >> 1, wave & 1, BigRing::kX128};
}

// Tile t of an item: weight matrix and 16-row feature block. Tiles
// 4 wn .. 4 wn + 3 belong to feature wave wn: for gate/up, 2 gate tiles then
// the 2 up tiles of the same 32 features; for down, 4 consecutive tiles.
template <int NMAT>
__device__ __forceinline__ void tile_of(int t, int g, int hs, int& m, int& fb) {
    if (NMAT == 2) {
        m = (t & 3) >> 1;
        fb = g * (hs ? 16 : 8) + (t >> 2) * 2 + (t & 1);
    } else {
        m = 0;
        fb = g * (hs ? 32 : 16) + t;
    }
}

// DMA sources of one item at K-group 0; group kg adds kg times the per-group
// stride of each stream. The weight-tile bases and LDS targets are
// wave-uniform (SGPRs); the per-lane parts are 32-bit element offsets to keep
// the loop's VGPRs low.
struct IssuePtrs {
    const uint4* w[4];       // this wave's weight tiles (2 or 4; lane added at issue)
    const uint16_t* s;       // wave 0: 16 B of scales of this lane
    uint32_t g;              // waves 1, 2: gsum offset of one row
    uint32_t x[4];           // src offset of 16 B of one activation row, per row DMA (4 or 2)
    int hs;
};

template <int NMAT>
__device__ __forceinline__ IssuePtrs issue_ptrs(const BigArgs& a, const BigItem& it, int K, int KG,
                                                int wave, int lane) {
    using RG = BigRing;
    IssuePtrs p;
    const bool sh = it.e == a.E;
    const int hs = it.hs;
    p.hs = hs;
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
    // Weight DMA j of this wave fills tile nw * wave + j (nw = 2 or 4).
    const int nw = hs ? 4 : 2;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int m, fb;
        tile_of<NMAT>(wave * nw + (j < nw ? j : 0), it.g, hs, m, fb);
        p.w[j] = wbase[m] + (size_t)fb * KG * 64;
    }
    // Scales (wave 0): lane l fetches half l % 2 (16 B) of tile l / 2's 32 B;
    // a 128-row item has 16 tiles, so lanes 32-63 fetch them a second time.
    {
        int m, fb;
        tile_of<NMAT>((lane >> 1) & (hs ? 31 : 15), it.g, hs, m, fb);
        p.s = sbase[m] + (size_t)fb * KG * 16 + (lane & 1) * 8;
    }
    // Row group sums (waves 1, 2): row 64 (wave - 1) + lane (a 64-row item
    // uses rows 0-63; rows past the tile's end repeat row 0).
    p.g = lds_read32(it.tab + 16 + (((wave - 1) & 1) * 64 + lane) * 4) * (uint32_t)KG;
    // Activation DMA j fills rows rpw * wave + 4 j + lane / 16 (rpw = 16 or 8
    // rows per wave); lane's LDS slot lane % 16 holds chunk (lane % 16) ^
    // (row & 15) of its row. The table's row map holds the token (gate/up) or
    // the grouped row (down) of each tile row; rows past the tile's end
    // repeat row 0.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = (hs ? wave * 8 : wave * 16) + j * 4 + (lane >> 4);
        p.x[j] = lds_read32(it.tab + 16 + row * 4) * (uint32_t)K +
                 (uint32_t)((lane & 15) ^ (row & 15)) * 8;
    }
    return p;
}

// Exactly kDma DMAs per wave: group kg of the item into `slot`. DMAs 0-1
// are weight tiles and 2-3 activation rows in both shapes; 4-5 are weight
// tiles 2-3 (64-row item) or activation DMAs 2-3 (128-row item), picked by a
// uniform select so that no DMA source is indexed dynamically.
__device__ __forceinline__ void big_issue(const BigArgs& a, const IssuePtrs& p, int kg, char* slot,
                                          int wave, int lane) {
    using RG = BigRing;
    const int hs = p.hs;
    const int nw = hs ? 4 : 2, nx = hs ? 2 : 4;
    const int xoff = hs ? RG::kX64 : RG::kX128;
#pragma unroll
    for (int j = 0; j < 2; ++j)
        dma16(p.w[j] + (size_t)kg * 64 + lane, slot + (wave * nw + j) * 1024);
#pragma unroll
    for (int j = 0; j < 2; ++j)
        dma16(a.src + (p.x[j] + (uint32_t)kg * 128), slot + xoff + (wave * nx + j) * RG::kQuad);
#pragma unroll
    for (int j = 2; j < 4; ++j) {
        const void* wsrc = p.w[j] + (size_t)kg * 64 + lane;
        const void* xsrc = a.src + (p.x[j] + (uint32_t)kg * 128);
        const int dst = hs ? (wave * 4 + j) * 1024 : RG::kX128 + (wave * 4 + j) * RG::kQuad;
        dma16(hs ? wsrc : xsrc, slot + dst);
    }
    if (wave == 0) dma16(p.s + (size_t)kg * 16, slot + RG::kSOff);
    else if (wave < 3) dma4(a.gsum + (p.g + (uint32_t)kg), slot + RG::kGOff + (wave - 1) * 256);
}

// Waits until at most N groups of this wave's DMAs are pending (the waves
// with a small DMA issue kDma + 1 per group).
template <int N>
__device__ __forceinline__ void big_wait_groups(bool small) {
    if (small) wait_vmcnt<N * (BigRing::kDma + 1)>();
    else wait_vmcnt<N * BigRing::kDma>();
}

// bf16 pair {hi(X), bf16(X - hi(X))} in the low dword of an MFMA A fragment
// (K slots 0, 1) for lanes 0-31; zero for lanes 32-63 (K slots 8-15).
__device__ __forceinline__ bf16x8 corr_a(float X, int h) {
    const float hi = __uint_as_float(__float_as_uint(X) & 0xffff0000u);
    const uint32_t v = pack_bf16x2(hi, X - hi);
    return __builtin_bit_cast(bf16x8, u32x4{h ? 0u : v, 0u, 0u, 0u});
}

// Operands a wave reads from one ring slot before its first MFMA: its weight
// fragments, their scales, the group sums of its rows and step 0's
// activation fragments. Issued one group ahead (see the main loop).
struct BigOps {
    u32x4 bw[2][2];
    uint32_t sc[2];
    float xs[2];
    u32x4 av0[2];
};

// A (activations): row R = wm*64 + tb*32 + col, chunk 8h + s for step s,
// stored at slot (8h + s) ^ (R & 15) = (8h ^ (col & 15)) ^ s. Rows are 256 B
// and the area is 256-B aligned, so step s's address is step 0's with bits
// 4-6 flipped by s; token block 1 is 32 rows (8 KiB) further.
__device__ __forceinline__ uint32_t big_xa0(const char* slot, const BigGeo& gm, int lane) {
    const int col = lane & 31, h = lane >> 5;
    return lds_addr(slot + gm.xoff) + (uint32_t)BigRing::row_off(gm.wm * 64 + col) +
           ((uint32_t)((8 * h) ^ (col & 15)) << 4);
}

// Issues the reads of BigOps (no wait).
__device__ __forceinline__ void big_load_ops(const char* slot, const BigGeo& gm, int lane, BigOps& o) {
    using RG = BigRing;
    const int wn = gm.wn, wm = gm.wm;
    const int col = lane & 31, h = lane >> 5;
    // B (weights): block jb = tiles 4 wn + 2 jb (+1 for features 16-31); the
    // lane's feature row col & 15 holds K chunks 8h .. 8h + 7 = packed-tile
    // lane slots q = 2h, 2h + 1, i.e. dword s of the pair is MFMA step s.
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
        const int t = wn * 4 + jb * 2 + (col >> 4);
        const uint32_t wa = lds_addr(slot + t * 1024) + (uint32_t)(((col & 15) + 32 * h) * 16);
        asm volatile("ds_read_b128 %0, %2\n ds_read_b128 %1, %2 offset:256"
                     : "=&v"(o.bw[jb][0]), "=&v"(o.bw[jb][1]) : "v"(wa));
        const uint32_t sa = lds_addr(slot + RG::kSOff + t * 32) + (uint32_t)((col & 15) * 2);
        asm volatile("ds_read_u16 %0, %1" : "=&v"(o.sc[jb]) : "v"(sa));
    }
    const uint32_t ga = lds_addr(slot + RG::kGOff) + (uint32_t)((wm * 64 + col) * 4);
    asm volatile("ds_read_b32 %0, %2\n ds_read_b32 %1, %2 offset:128"
                 : "=&v"(o.xs[0]), "=&v"(o.xs[1]) : "v"(ga));
    asm volatile("ds_read_b128 %0, %2\n ds_read_b128 %1, %2 offset:8192"
                 : "=&v"(o.av0[0]), "=&v"(o.av0[1]) : "v"(big_xa0(slot, gm, lane)));
}

// Waits for the reads of big_load_ops and consumes their registers. Every
// step calls it, whether or not the wave computes: an LDS read returns
// asynchronously, so a register the compiler thinks free after an unused
// read could be handed to another value and then overwritten by the late
// return (for example a store address), and a copy the compiler makes of an
// operand before the wait would read it too early.
__device__ __forceinline__ void big_wait_ops(BigOps& o) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(o.bw[0][0]), "+v"(o.bw[0][1]), "+v"(o.bw[1][0]), "+v"(o.bw[1][1]),
                   "+v"(o.sc[0]), "+v"(o.sc[1]), "+v"(o.xs[0]), "+v"(o.xs[1]), "+v"(o.av0[0]),
                   "+v"(o.av0[1]));
}

// One 128-K group of the wave's 64 x 64 tile: p = sum_k (128 + c) x - 136 X
// per 32 x 32 block (the caller applies the group's scales).
__device__ __forceinline__ void big_compute(const char* slot, const BigGeo& gm, int lane,
                                            const DqConst& dqc, BigOps& o, f32x16 (&p)[2][2]) {
    const int h = lane >> 5;
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(o.bw[0][0]), "+v"(o.bw[0][1]), "+v"(o.bw[1][0]), "+v"(o.bw[1][1]),
                   "+v"(o.sc[0]), "+v"(o.sc[1]), "+v"(o.xs[0]), "+v"(o.xs[1]), "+v"(o.av0[0]),
                   "+v"(o.av0[1]));
    // Seeds: -136 X per row, shared by both weight blocks.
    const bf16x8 bneg = __builtin_bit_cast(bf16x8, u32x4{0xC308C308u, 0u, 0u, 0u});
    f32x16 seed[2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) seed[tb] = mfma32x32x16(corr_a(o.xs[tb], h), bneg, f32x16{});

    const uint32_t xa0 = big_xa0(slot, gm, lane);
    u32x4 av[2][2];
    av[0][0] = o.av0[0];
    av[0][1] = o.av0[1];
    // Software pipeline per K-step s: the activation reads of s + 1 and the
    // int4 decode of s + 1 run under the MFMAs of s. sched_barrier keeps the
    // compiler from sinking the reads next to their wait (which would expose
    // the LDS latency every step).
    bf16x8 bv[2][2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) bv[0][jb] = dq_w4(o.bw[jb][0][0], dqc);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const int cb = s & 1, nb = cb ^ 1;
        if (s > 0) asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(av[cb][0]), "+v"(av[cb][1]));
        if (s < 7) {
            const uint32_t xs_addr = xa0 ^ (uint32_t)((s + 1) << 4);
            asm volatile("ds_read_b128 %0, %2\n ds_read_b128 %1, %2 offset:8192"
                         : "=&v"(av[nb][0]), "=&v"(av[nb][1]) : "v"(xs_addr));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int jb = 0; jb < 2; ++jb)
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
                p[jb][tb] = mfma32x32x16(as_bf16x8(av[cb][tb]), bv[cb][jb], s == 0 ? seed[tb] : p[jb][tb]);
        if (s < 7) {
#pragma unroll
            for (int jb = 0; jb < 2; ++jb) bv[nb][jb] = dq_w4(o.bw[jb][(s + 1) >> 2][(s + 1) & 3], dqc);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// acc += scale_col * p (one fma per element).
__device__ __forceinline__ void big_rescale(const uint32_t (&sc)[2], const f32x16 (&p)[2][2],
                                            f32x16 (&acc)[2][2]) {
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
        const float scale = bf16_to_f32(sc[jb]);
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[jb][tb][i] = __builtin_fmaf(scale, p[jb][tb][i], acc[jb][tb][i]);
    }
}

// Row (0..127) of accumulator element i of token block tb for wave row half wm.
__device__ __forceinline__ int acc_row(int wm, int tb, int i, int h) {
    return wm * 64 + tb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
}

// One step of the recursive-halving lane reduction over the first 2N values.
template <int N>
__device__ __forceinline__ void halve(float (&v)[32], int col) {
    const bool upper = (col & N) != 0;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        const float send = upper ? v[j] : v[j + N];
        const float keep = upper ? v[j + N] : v[j];
        v[j] = keep + __shfl_xor(send, N);
    }
}

template <int NMAT>
__device__ __forceinline__ void big_epilogue(const BigArgs& a, const BigItem& cur, char* lds,
                                             const BigGeo& gm, int lane, f32x16 (&acc)[2][2]) {
    const int wn = gm.wn, wm = gm.wm;
    const int hs = cur.hs;
    // Laundered lane index: keeps the compiler from hoisting the per-row
    // addresses below out of the streaming loop (they would stay live across
    // it and spill).
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int col = ln & 31, h = ln >> 5;
    if constexpr (NMAT == 2) {
        // h = silu(g) * u (bf16) for this lane's feature and 32 rows; then the
        // sum of the rounded h over the workgroup's 128 features (one group of
        // I) per row: a fixed butterfly over the 32 lanes of the wave that
        // share rows, then the 4 feature waves in order. A 64-row item's 8
        // waves cover two such groups, waves 0-3 and 4-7.
        uint16_t* hbase = a.h + (size_t)cur.r0 * a.I + cur.g * (hs ? 256 : 128) + wn * 32;
        float v[32];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                const uint32_t hb = pack_bf16x2(silu_fast(acc[0][tb][i]) * acc[1][tb][i],
                                                silu_fast(acc[0][tb][i + 1]) * acc[1][tb][i + 1]);
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int lr = acc_row(wm, tb, i + e, h);
                    const uint32_t he = e ? hb >> 16 : hb & 0xffffu;
                    if (lr < cur.nr) hbase[lr * a.I + col] = (uint16_t)he;
                    v[tb * 16 + i + e] = bf16_to_f32(he);
                }
            }
        // Recursive halving: after the step with lane mask m the lane keeps the
        // half of its values whose index bit matches (col & m); at the end lane
        // col holds the 32-lane sum of value index col.
        halve<16>(v, col);
        halve<8>(v, col);
        halve<4>(v, col);
        halve<2>(v, col);
        halve<1>(v, col);
        const uint32_t red = lds_addr(lds + BigRing::kRed);
        const int myrow = acc_row(wm, col >> 4, col & 15, h);
        const int rstride = hs ? 64 : kBigRows;   // rows of the item
        lds_write32(red + (uint32_t)((wn * rstride + myrow) * 4), v[0]);
        __builtin_amdgcn_s_barrier();
        if ((wn & 3) == 0) {
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w)
                s += __uint_as_float(lds_read32(red + (uint32_t)(((wn + w) * rstride + myrow) * 4)));
            const int grp = hs ? cur.g * 2 + (wn >> 2) : cur.g;
            if (myrow < cur.nr) a.hsum[((size_t)cur.r0 + myrow) * (a.I / 128) + grp] = s;
        }
        __builtin_amdgcn_s_barrier();   // partials consumed before the next item reuses them
    } else {
        // Per-row expert outputs as bf16 (the combine adds them in fp32):
        // half the bytes of the largest write and read of a prefill layer.
        uint16_t* d16 = reinterpret_cast<uint16_t*>(a.dpart);
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
            uint16_t* dbase = d16 + (size_t)cur.r0 * a.H + cur.g * (hs ? 512 : 256) + wn * 64 + jb * 32;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int lr = acc_row(wm, tb, i, h);
                    if (lr < cur.nr) dbase[lr * a.H + col] = (uint16_t)(pack_bf16x2(acc[jb][tb][i], 0.0f) & 0xffffu);
                }
        }
    }
}

#define BIG_T(i) do {} while (0)

template <int NMAT>
__global__ __launch_bounds__(512) void w4_big_kernel(BigArgs a) {
    using RG = BigRing;
    extern __shared__ __align__(16) char lds[];
    const DqConst dqc = dq_const();
    int* table = reinterpret_cast<int*>(lds + RG::kTab);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool small = wave < 3;   // issues one small DMA per group
    const int K = NMAT == 2 ? a.H : a.I;
    const int KG = K / 128;
    const int nfg = (NMAT == 2 ? a.I : a.H) / BigShape<NMAT>::kFeat;
    // ntiles[1]: tiles taken as 128-row items; the rest are half tiles.
    const int ntiles = a.ntiles[0], n128 = a.ntiles[1];
    const long total = big2_total(ntiles, n128, nfg);
    const long nitems = big_rounds(total);

    for (long k0 = 0; k0 < nitems; k0 += kBigTable) {
        const int cnt = (int)min((long)kBigTable, nitems - k0);
        big2_fill_table<NMAT == 2>(a.tiles, a.rows_tok, table, k0, cnt, nfg, n128);
        __syncthreads();
        const long nsteps = (long)cnt * KG;

        // Ring of kBigD slots; group g lives in slot g % kBigD. Per group:
        // compute g; wait for g + 1's DMA and barrier (every wave is then done
        // with slot g, and g + 1 is visible); refill slot g with group
        // g + kBigD; issue the reads of g + 1's operands; apply g's scales
        // while those reads are in flight.
        int iss_k = 0, iss_g = 0;
        IssuePtrs iss = issue_ptrs<NMAT>(a, big_item(lds + RG::kTab, 0), K, KG, wave, lane);
        auto issue_next = [&](long g) {
            big_issue(a, iss, iss_g, lds + (g % kBigD) * RG::kSlot, wave, lane);
            if (++iss_g == KG) {
                iss_g = 0;
                if (++iss_k < cnt)
                    iss = issue_ptrs<NMAT>(a, big_item(lds + RG::kTab, iss_k), K, KG, wave, lane);
            }
        };
        for (int j = 0; j < kBigD; ++j)
            if (j < nsteps) issue_next(j);
        if (nsteps >= 3) big_wait_groups<2>(small);
        else if (nsteps == 2) big_wait_groups<1>(small);
        else wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        int cur_k = 0, cur_g = 0;
        BigItem cur = big_item(lds + RG::kTab, 0);
        BigGeo gc = big_geo(cur.hs, wave);
        BigOps ops;
        big_load_ops(lds, gc, lane, ops);
        big_wait_ops(ops);
        // Whether this wave's 64 rows hold any live row (wave-uniform per item).
        bool live = cur.nr > gc.wm * 64;
        f32x16 acc[2][2];
#pragma unroll
        for (int jb = 0; jb < 2; ++jb)
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) acc[jb][tb] = f32x16{};

        for (long step = 0; step < nsteps; ++step) {
            f32x16 p[2][2];
            // A wave whose 64 rows are all past the tile's end skips the group;
            // a half-live wave computes both 32-row blocks (one branch-free body
            // keeps the accumulators in fixed registers).
            if (live) big_compute(lds + (step % kBigD) * RG::kSlot, gc, lane, dqc, ops, p);
            BIG_T(0);
            if (step + 2 < nsteps) big_wait_groups<1>(small);
            else wait_vmcnt<0>();
            BIG_T(1);
            __builtin_amdgcn_s_barrier();
            BIG_T(2);
            if (step + kBigD < nsteps) issue_next(step + kBigD);
            const uint32_t sc[2] = {ops.sc[0], ops.sc[1]};
            if (step + 1 < nsteps) {
                // Group step + 1 may start the next item, of the other shape.
                const BigGeo gn = cur_g + 1 < KG ? gc : big_geo(big_item(lds + RG::kTab, cur_k + 1).hs, wave);
                big_load_ops(lds + ((step + 1) % kBigD) * RG::kSlot, gn, lane, ops);
            }
            BIG_T(3);
            if (live) big_rescale(sc, p, acc);
            BIG_T(4);
            if (++cur_g == KG) {
                big_epilogue<NMAT>(a, cur, lds, gc, lane, acc);
#pragma unroll
                for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                    for (int tb = 0; tb < 2; ++tb) acc[jb][tb] = f32x16{};
                cur_g = 0;
                if (++cur_k < cnt) {
                    cur = big_item(lds + RG::kTab, cur_k);
                    gc = big_geo(cur.hs, wave);
                    live = cur.nr > gc.wm * 64;
                }
            }
            // Last in the iteration: the next step's operands have arrived
            // before anything (including copies the compiler makes for the
            // loop) reads their registers.
            big_wait_ops(ops);
            BIG_T(5);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
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
