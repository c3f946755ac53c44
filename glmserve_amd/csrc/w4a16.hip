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
#include <utility>
#include "common.hpp"
#include "dispatch.hpp"
#include "kernels.hpp"
#include "topk.hpp"

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
// Grouped expert products (decode / small-group regime).
//
// One kernel template serves both projections:
//   NMAT = 2: gate and up of the same 16 features, SiLU(g) * u epilogue,
//             B operand = activation rows gathered through rows_tok;
//   NMAT = 1: down, B operand = the contiguous grouped h rows.
// Lane l: r = l & 15 is both the weight row (A operand) and the token column
// (B operand / output column); q = l >> 4 selects the 32-K quarter of each
// 128-K tile. MFMA step d (0..3) covers K = 32q + 8d + [0,8) for this lane.
// Output lane layout: rows 4q + j (j = 0..3), column r.
//
// Work. A workgroup of 8 waves takes one tile (up to 16 grouped rows of one
// expert) and 8 consecutive 16-row weight blocks of it, one per wave; the
// activation rows the tile needs are streamed once for all 8 waves.
//
// Streaming. Everything a batch of PF 128-K groups needs -- each wave's
// weight tiles and scales, and the tile's 16 activation rows -- is copied
// global -> LDS by the LDS-DMA path (global_load_lds_dwordx4 / _dword), so
// nothing in flight occupies registers. A ring of D batch slots keeps D-1
// batches in flight. Every wave issues the same number of DMA instructions
// per batch (kDma), so "batch b has landed" is the immediate
// s_waitcnt vmcnt(kDma * (D - 2)); one s_barrier per batch then publishes the
// shared rows and frees the oldest slot. The pipeline runs across work items,
// so it never drains between them. LDS reads are inline ds_read_b128 with
// their own lgkmcnt wait, which keeps the compiler from inserting a vmcnt(0)
// for the pending DMA. Their outputs are early-clobber: a read returns
// asynchronously, so no output may share a register with an address still
// needed by a later read.
//
// Activation rows sit at a stride of PF * 256 B in a slot, so each DMA's 64
// lanes read whole rows (consecutive lanes, consecutive 16 B: full-speed L2
// coalescing). Inside a row, 16-byte chunk c is stored at slot c ^ (r & 15),
// which puts the 16 rows an MFMA B fragment reads at one chunk on 16
// distinct bank groups.
//
// The group sum X_j = sum_k x[k][j] that removes the +136 bias of the int4
// decode comes from one more MFMA against an all-ones A operand.
// ---------------------------------------------------------------------------
struct ExpArgs {
    const uint4* wq[2];      // routed experts, stacked native matrices
    const uint16_t* ws[2];
    const uint4* swq[2];     // shared expert
    const uint16_t* sws[2];
    const uint16_t* src;     // x [n, H] (NMAT = 2) or h [R, I] (NMAT = 1)
    const float* gsum;       // group sums of src rows: xsum [n, H/128] or hsum [R, I/128]
    const int4* tiles; const int* ntiles; const int* rows_tok;
    uint16_t* h; float* hsum; float* dpart;
    unsigned int* tick; float* tpart; int tcap;   // tail split state (gate/up stream kernel)
    int H, I, E;
    FusedRoute route;        // route.cs != null: select and dispatch first (gate/up stream kernel)
};


template <int NMAT, int PF, int D, int NW>
struct Ring {
    static_assert(PF == 1 || PF == 2 || PF == 4, "a batch row span is 256, 512 or 1024 bytes");
    static constexpr int kW = 1024;                               // one weight tile
    static constexpr int kWBytes = NW * NMAT * PF * kW;    // all waves' tiles
    static constexpr int kSBytes = NW * 256;               // scale dwords per wave
    static constexpr int kRS = PF * 256;                          // activation row stride
    static constexpr int kXBytes = kTileRows * kRS;
    static constexpr int kCPR = 16 * PF;                          // 16-B chunks per row
    static constexpr int kRPD = 64 / kCPR;                        // rows per activation DMA
    static constexpr int kNX = kTileRows / kRPD;                  // activation DMAs per batch
    // Activation DMAs per wave; with fewer DMAs than waves, the waves past
    // them issue one placeholder DMA into kJunk so every wave issues kDma.
    static constexpr int kXDma = kNX >= NW ? kNX / NW : 1;
    static_assert(kNX < NW || kXDma * NW == kNX, "activation DMAs split evenly");
    static constexpr int kJunkBytes = kNX < NW ? 1024 : 0;
    // Group sums X[i][r] of the batch's PF groups and 16 rows (256 B), and
    // the target of the other waves' placeholder group-sum DMA.
    static constexpr int kGOff = kWBytes + kSBytes + kXBytes + kJunkBytes;
    static constexpr int kSlot = kGOff + 512;
    static constexpr int kBytes = D * kSlot;
    static constexpr int kRed = kBytes;                               // [NW][16] h group-sum partials
    static constexpr int kTotal = kRed + NW * 64 + kTable * kTabInts * 4;   // + the item table
    static_assert(kTotal * (8 / NW) <= 160 * 1024, "8 / NW workgroups per CU");
    static constexpr int kDma = NMAT * PF + 2 + kXDma;            // DMA instructions per batch per wave
};

// Work items of a workgroup come in steps k: WG-item base + k * nwg is
// (tile, block group), and wave w takes weight block 8 * group + w. A chunk of
// up to kTable steps is described in an LDS table read back with inline
// ds_read (no vector-memory loads inside the pipeline, whose waits would
// drain the DMA queue): per step {expert, row0, nrows, block group} and the 16
// token ids of the tile rows (row 0's token past nrows).

struct Item {
    const uint4* wq[2];
    const uint16_t* ws[2];
    int r0, nr, fb;
    uint32_t tok[2];   // src row of this lane in each of this wave's activation DMAs
    uint32_t gtok;     // gsum row of tile row lane % 16
};

template <int NMAT, int PF, int D, int NW>
__device__ __forceinline__ Item item_from_table(const ExpArgs& a, const int* table, int k,
                                                int wave, int lane, int nfb, int KG) {
    using RG = Ring<NMAT, PF, D, NW>;
    const uint32_t base = lds_addr(table + k * kTabInts);
    const uint4 h = lds_bcast16(base);
    Item it;
    const int e = sgpr(h.x);
    it.r0 = sgpr(h.y);
    it.nr = sgpr(h.z);
    it.fb = sgpr(h.w) * NW + wave;
    // Activation DMA j of this wave covers tile rows (wave * kXDma + j) * kRPD + [0, kRPD);
    // this lane's row is the lane / kCPR-th of them.
#pragma unroll
    for (int j = 0; j < RG::kXDma; ++j) {
        const int row = ((wave * RG::kXDma + j) * RG::kRPD + lane / RG::kCPR) % kTileRows;
        if (NMAT == 2) it.tok[j] = lds_read_u32(base + 16 + row * 4);
        else it.tok[j] = (uint32_t)(it.r0 + (row < it.nr ? row : 0));
    }
    {
        const int row = lane & 15;
        it.gtok = NMAT == 2 ? lds_read_u32(base + 16 + row * 4)
                            : (uint32_t)(it.r0 + (row < it.nr ? row : 0));
    }
    const bool sh = e == a.E;
    const size_t mstride_q = (size_t)nfb * KG * 64;   // uint4 per matrix
    const size_t mstride_s = (size_t)nfb * KG * 16;   // u16 per matrix
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const int mm = m < NMAT ? m : 0;
        it.wq[m] = (sh ? a.swq[mm] : a.wq[mm] + (size_t)e * mstride_q) + (size_t)it.fb * KG * 64;
        it.ws[m] = (sh ? a.sws[mm] : a.ws[mm] + (size_t)e * mstride_s) + (size_t)it.fb * KG * 16;
    }
    return it;
}

// Fills table steps [k0, k0 + cnt) (whole workgroup; ordinary loads; the
// caller has drained all DMA and synchronizes afterwards).
__device__ __forceinline__ void fill_table(const ExpArgs& a, int* table, int base, int nwg,
                                           int ngrp, int k0, int cnt) {
    for (int i = threadIdx.x; i < cnt * kTabInts; i += blockDim.x) {
        const int k = i / kTabInts, f = i % kTabInts;
        const int item = base + (k0 + k) * nwg;
        const int4 tile = a.tiles[item / ngrp];
        int v;
        if (f == 0) v = tile.x;
        else if (f == 1) v = tile.y;
        else if (f == 2) v = tile.z;
        else if (f == 3) v = (int)(item % ngrp);
        else {
            const int row = f - 4;
            v = a.rows_tok ? a.rows_tok[tile.y + (row < tile.z ? row : 0)] : 0;
        }
        table[i] = v;
    }
}

// Issues batch bb of item `it` into ring slot `slot` (exactly kDma DMAs).
template <int NMAT, int PF, int D, int NW>
__device__ __forceinline__ void issue_batch(const ExpArgs& a, const Item& it, int bb, int K,
                                            int KG, char* slot, int wave, int lane) {
    using RG = Ring<NMAT, PF, D, NW>;
    const int kg0 = bb * PF;
    // Weight tiles: [wave][m][i] 1 KiB each, lane-contiguous like the global tile.
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int i = 0; i < PF; ++i) {
            const int kg = min(kg0 + i, KG - 1);
            dma16(it.wq[m] + (size_t)kg * 64 + lane, slot + ((wave * NMAT + m) * PF + i) * RG::kW);
        }
    // Scales: lane l < NMAT*PF*8 fetches dword (l % 8) of group (l / 8) % PF of matrix
    // l / (PF*8); the 16 bf16 scales of a (matrix, group) are 8 dwords.
    {
        const int m = min(lane / (PF * 8), NMAT - 1);
        const int d = lane % (PF * 8);
        const int kg = min(kg0 + d / 8, KG - 1);
        dma4(it.ws[m] + (size_t)kg * 16 + (d % 8) * 2, slot + RG::kWBytes + wave * 256);
    }
    // Group sums: wave 0 lane l fetches X of tile row l % 16, group kg0 + l / 16.
    {
        const int kg = min(kg0 + (lane >> 4) % PF, KG - 1);
        dma4(a.gsum + (size_t)it.gtok * KG + kg, slot + RG::kGOff + (wave == 0 ? 0 : 256));
    }
    // Activation rows: whole rows per DMA, chunk slot p of a row holds chunk
    // p ^ (row & 15) of the batch's PF * 128 K (row r0 stands in past nr;
    // those token columns are computed but never stored).
#pragma unroll
    for (int j = 0; j < RG::kXDma; ++j) {
        const int blk = wave * RG::kXDma + j;
        const int row = (blk * RG::kRPD + lane / RG::kCPR) % kTileRows;
        const int c = (lane % RG::kCPR) ^ (row & 15);
        const int koff = min(kg0 * 128 + c * 8, K - 8);
        char* dst = blk < RG::kNX ? slot + RG::kWBytes + RG::kSBytes + blk * 1024
                                  : slot + RG::kWBytes + RG::kSBytes + RG::kXBytes;
        dma16(a.src + (size_t)it.tok[j] * K + koff, dst);
    }
}

// One 128-K group's LDS operands of a wave: its 4 activation fragments
// (the 16 token columns), its weight tile(s), their 4 row scales and the
// group sum of its token column.
struct ExpOps {
    u32x4 x[4], w[2];
    u32x2 s[2];
    float g;
};

// Issues the reads of group i of the batch in `slot` (no wait).
template <int NMAT, int PF, int D, int NW>
__device__ __forceinline__ void exp_load_ops(const char* slot, int i, int wave, int lane,
                                             ExpOps& o) {
    using RG = Ring<NMAT, PF, D, NW>;
    const int r = lane & 15, q = lane >> 4;
    const uint32_t wa = lds_addr(slot) + (uint32_t)(wave * NMAT * PF * RG::kW + lane * 16) + i * RG::kW;
    const uint32_t sa = lds_addr(slot + RG::kWBytes + wave * 256) + (uint32_t)(q * 8) + i * 32;
    // Chunk 16 i + 4 q + d of row r is at r * kRS + 256 i + 16 ((4 q + d) ^ r).
    const uint32_t xrow = lds_addr(slot + RG::kWBytes + RG::kSBytes) + (uint32_t)(r * RG::kRS + 256 * i);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t xa = xrow + (uint32_t)(((4 * q + d) ^ r) * 16);
        asm volatile("ds_read_b128 %0, %1" : "=&v"(o.x[d]) : "v"(xa));
    }
    const uint32_t ga = lds_addr(slot + RG::kGOff) + (uint32_t)((i * 16 + r) * 4);
    asm volatile("ds_read_b32 %0, %1" : "=&v"(o.g) : "v"(ga));
    if constexpr (NMAT == 2) {
        asm volatile("ds_read_b128 %0, %2\n ds_read_b128 %1, %2 offset:%c3"
                     : "=&v"(o.w[0]), "=&v"(o.w[1]) : "v"(wa), "i"(PF * RG::kW));
        asm volatile("ds_read_b64 %0, %2\n ds_read_b64 %1, %2 offset:%c3"
                     : "=&v"(o.s[0]), "=&v"(o.s[1]) : "v"(sa), "i"(PF * 32));
    } else {
        asm volatile("ds_read_b128 %0, %1" : "=&v"(o.w[0]) : "v"(wa));
        asm volatile("ds_read_b64 %0, %1" : "=&v"(o.s[0]) : "v"(sa));
    }
}

__device__ __forceinline__ void exp_wait_ops(ExpOps& o) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(o.x[0]), "+v"(o.x[1]), "+v"(o.x[2]), "+v"(o.x[3]), "+v"(o.w[0]),
                   "+v"(o.w[1]), "+v"(o.s[0]), "+v"(o.s[1]), "+v"(o.g));
}

// The PF groups of one batch.
template <int PF>
struct BatchOps {
    ExpOps g[PF];
};

template <int NMAT, int PF, int D, int NW>
__device__ __forceinline__ void exp_load_batch(const char* slot, int wave, int lane,
                                               BatchOps<PF>& b) {
#pragma unroll
    for (int i = 0; i < PF; ++i) exp_load_ops<NMAT, PF, D, NW>(slot, i, wave, lane, b.g[i]);
}

template <int PF>
__device__ __forceinline__ void exp_wait_batch(BatchOps<PF>& b) {
    // One wait for all reads; the per-group asm statements only tie each
    // group's registers to it.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < PF; ++i) exp_wait_ops(b.g[i]);
}

// A batch's groups in one basic block, so the int4 decode of one group can be
// scheduled under another group's MFMAs:
// acc[m] += scale * (sum_k (128 + c) x - 136 X) per group, X the group sum of
// the token column.
template <int NMAT, int PF>
__device__ __forceinline__ void exp_compute_batch(const BatchOps<PF>& b, const DqConst& dqc,
                                                  f32x4 (&acc)[NMAT]) {
    f32x4 p[PF][NMAT];
#pragma unroll
    for (int i = 0; i < PF; ++i)
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
                p[i][m] = mfma16x16x32(dq_w4(b.g[i].w[m][d], dqc), as_bf16x8(b.g[i].x[d]),
                                       d == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : p[i][m]);
#pragma unroll
    for (int i = 0; i < PF; ++i) {
        const float off = -136.0f * b.g[i].g;
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            const u32x2 sv = b.g[i].s[m];
            const float sc[4] = {bf16_to_f32(sv.x & 0xffffu), __uint_as_float(sv.x & 0xffff0000u),
                                 bf16_to_f32(sv.y & 0xffffu), __uint_as_float(sv.y & 0xffff0000u)};
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[m][j] = __builtin_fmaf(sc[j], p[i][m][j] + off, acc[m][j]);
        }
    }
}

template <int NMAT, int PF, int D, int NW>
__global__ __launch_bounds__(NW * 64) void w4_expert_kernel(ExpArgs a) {
    using RG = Ring<NMAT, PF, D, NW>;
    extern __shared__ __align__(16) char ring[];
    const DqConst dqc = dq_const();
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;
    const int K = NMAT == 2 ? a.H : a.I;
    const int KG = K / 128;
    const int nfb = (NMAT == 2 ? a.I : a.H) / 16;
    const int ngrp = nfb / NW;
    const int nbatch = KG / PF;   // the launcher picks PF dividing KG
    const int total = *a.ntiles * ngrp;
    const int nwg = (int)gridDim.x;
    const int base = (int)blockIdx.x;
    const int nitems = base < total ? (total - base + nwg - 1) / nwg : 0;
    int* table = reinterpret_cast<int*>(ring + RG::kRed + NW * 64);
    // Steps per unrolled block: a multiple of the ring depth (constant slot
    // addresses) and of 2 (the two operand buffers alternate).
    constexpr int kU = (D % 2 == 0) ? D : 2 * D;

    for (int k0 = 0; k0 < nitems; k0 += kTable) {
        const int cnt = min(kTable, nitems - k0);
        fill_table(a, table, base, nwg, ngrp, k0, cnt);
        __syncthreads();
        const int nsteps = cnt * nbatch;

        // Ring of D batch slots; batch b lives in slot b % D. The prologue
        // fills every slot. Per batch b, with its operands already read into
        // registers: wait for batch b + 1 and barrier (every wave is then done
        // reading slot b, and b + 1 is visible), refill slot b with batch
        // b + D, issue the reads of b + 1's operands, then compute b under
        // those reads.
        int iss_k = 0, iss_b = 0;
        Item iss = item_from_table<NMAT, PF, D, NW>(a, table, 0, wave, lane, nfb, KG);
        auto issue_next = [&](char* slot) {
            issue_batch<NMAT, PF, D, NW>(a, iss, iss_b, K, KG, slot, wave, lane);
            if (++iss_b == nbatch) {
                iss_b = 0;
                if (++iss_k < cnt)
                    iss = item_from_table<NMAT, PF, D, NW>(a, table, iss_k, wave, lane, nfb, KG);
            }
        };
#pragma unroll
        for (int j = 0; j < D; ++j)
            if (j < nsteps) issue_next(ring + j * RG::kSlot);
        if (nsteps >= D) wait_vmcnt<RG::kDma * (D - 1)>();
        else wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        BatchOps<PF> ops[2];
        exp_load_batch<NMAT, PF, D, NW>(ring, wave, lane, ops[0]);

        int cur_k = 0, cur_b = 0;
        Item cur = item_from_table<NMAT, PF, D, NW>(a, table, 0, wave, lane, nfb, KG);
        f32x4 acc[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};

        for (int step0 = 0; step0 < nsteps; step0 += kU) {
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int step = step0 + u;
            if (step >= nsteps) break;
            BatchOps<PF>& now = ops[u & 1];
            exp_wait_batch<PF>(now);
            // Batch step + 1 has landed once at most the batches issued after
            // it (up to step + D - 1) are pending.
            if (step + D - 1 < nsteps) wait_vmcnt<RG::kDma * (D - 2)>();
            else wait_vmcnt<0>();
            __builtin_amdgcn_s_barrier();
            if (step + D < nsteps) issue_next(ring + (u % D) * RG::kSlot);
            if (step + 1 < nsteps)
                exp_load_batch<NMAT, PF, D, NW>(ring + ((u + 1) % D) * RG::kSlot, wave, lane,
                                                ops[(u + 1) & 1]);
            exp_compute_batch<NMAT, PF>(now, dqc, acc);
            if (++cur_b == nbatch) {
                const bool valid = r < cur.nr;
                const size_t row = (size_t)cur.r0 + r;
                if constexpr (NMAT == 2) {
                    static_assert(NMAT == 1 || NW == 8, "a workgroup step covers one 128-feature group");
                    const uint32_t h01 = pack_bf16x2(silu_fast(acc[0][0]) * acc[1][0],
                                                     silu_fast(acc[0][1]) * acc[1][1]);
                    const uint32_t h23 = pack_bf16x2(silu_fast(acc[0][2]) * acc[1][2],
                                                     silu_fast(acc[0][3]) * acc[1][3]);
                    if (valid)
                        *reinterpret_cast<uint2*>(a.h + row * a.I + cur.fb * 16 + 4 * q) =
                            uint2{h01, h23};
                    // hsum of the rounded h over the step's 128 features (one
                    // group of I) per tile row: 4 features per lane, the 4 row
                    // quarters, then the 8 waves in order.
                    float ps = (bf16_to_f32(h01 & 0xffffu) + __uint_as_float(h01 & 0xffff0000u)) +
                               (bf16_to_f32(h23 & 0xffffu) + __uint_as_float(h23 & 0xffff0000u));
                    ps = ps + __shfl_xor(ps, 16);
                    ps = ps + __shfl_xor(ps, 32);
                    const uint32_t red = lds_addr(ring + RG::kRed);
                    if (q == 0) lds_write_f32(red + (uint32_t)((wave * 16 + r) * 4), ps);
                    __builtin_amdgcn_s_barrier();
                    if (wave == 0 && q == 0) {
                        float tot = 0.0f;
#pragma unroll
                        for (int w = 0; w < NW; ++w)
                            tot += __uint_as_float(lds_read_u32(red + (uint32_t)((w * 16 + r) * 4)));
                        if (valid) a.hsum[row * (a.I / 128) + cur.fb / NW] = tot;
                    }
                    __builtin_amdgcn_s_barrier();   // partials consumed before reuse
                } else {
                    if (valid)
                        *reinterpret_cast<float4*>(a.dpart + row * a.H + cur.fb * 16 + 4 * q) =
                            make_float4(acc[0][0], acc[0][1], acc[0][2], acc[0][3]);
                }
#pragma unroll
                for (int m = 0; m < NMAT; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
                cur_b = 0;
                if (++cur_k < cnt)
                    cur = item_from_table<NMAT, PF, D, NW>(a, table, cur_k, wave, lane, nfb, KG);
            }
        }
        }
        // All DMA has landed (the last step waited vmcnt(0)); every wave is
        // done reading the ring and the table before the next chunk refills.
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Streaming decode kernel (K-group count a multiple of 16): the same work
// decomposition and arithmetic as w4_expert_kernel, with the two streams
// decoupled.
//   * Weights and scales are private to a wave: each wave loads its own
//     tiles straight into registers (global_load_dwordx4 of the 1 KiB tile:
//     lane l gets bytes 16 l .. 16 l + 15, exactly its MFMA A operand),
//     SP groups ahead, with no LDS staging and no barrier.
//   * The tile's activation rows and group sums, shared by the 8 waves, come
//     through LDS in batches of 16 K-groups (64 KiB + 1 KiB) by LDS-DMA into
//     two buffers; one barrier per batch. Batch b + 1 is issued half-way
//     through batch b.
// All loads complete in issue order, so every wait is an immediate vmcnt:
// the number of loads issued after the one waited for (counted statically in
// the 16-group unrolled batch body).
// ---------------------------------------------------------------------------
constexpr int kSGB = 16;     // K-groups per activation batch
constexpr int kSActDma = 9;  // activation + group-sum DMAs per wave per batch
constexpr int kSPGU = 4;
constexpr int kSPDown = 8;

// Stream table step: {expert, row0, nrows, block group}, the 16 token ids,
// then {first batch, batches, tail item or -1, 0}.
constexpr int kSTabInts = 24;

// Work schedule. An item (tile, block group) covers all K in BPI batches of
// 16 groups; its result is the batch totals added in batch order,
// T = ((t_0 + t_1) + t_2) ..., each t_b accumulated from zero. After R full
// rounds of items over the workgroups, the rem items left over would keep rem
// workgroups busy for a whole item while the rest idle; when splitting them
// by batch shortens that last round, each of their batches is a unit of its
// own (a "part"). A part stores t_b; at the end of the kernel the workgroup
// that holds an item's last part (by ticket) adds the stored t_b in batch
// order and finishes the item. Whole or split, an item's arithmetic is the
// same, so results do not depend on how a batch's work was spread.
// The tickets (kTailTicks, zero at launch: the call's router or dispatch kernel clears them) and the
// stored t_b ([part][value][thread], 16 KiB per part, room for a.tcap parts)
// are in the caller's workspace; a split needs rem <= kTailTicks items and
// rem * BPI <= a.tcap parts.
constexpr int kTailPartBytes = 8 * 512 * 4;

struct SSched {
    int R, rem, split, nunits;
};

__device__ __forceinline__ SSched s_sched(int total, int nwg, int base, int BPI, int tcap) {
    SSched sc;
    sc.R = total / nwg;
    sc.rem = total - sc.R * nwg;
    const int parts = sc.rem * BPI;
    // With no full round (a handful of items) the split's ticket and
    // finishing cost more than the shorter round saves.
    sc.split = BPI > 1 && sc.R > 0 && sc.rem > 0 && sc.rem <= kTailTicks && parts <= tcap &&
               (parts + nwg - 1) / nwg < BPI;
    if (sc.split)
        sc.nunits = sc.R + (base < parts ? (parts - base + nwg - 1) / nwg : 0);
    else
        sc.nunits = base < total ? (total - base + nwg - 1) / nwg : 0;
    return sc;
}

// Unit u of workgroup `base`: item, first batch, batches, tail item (-1: whole).
__device__ __forceinline__ int4 s_unit(const SSched& sc, int base, int nwg, int BPI, int u) {
    if (sc.split && u >= sc.R) {
        const int t = base + (u - sc.R) * nwg;
        return int4{sc.R * nwg + t / BPI, t % BPI, 1, t / BPI};
    }
    return int4{base + u * nwg, 0, BPI, -1};
}

// Fills stream-table steps [k0, k0 + cnt) (whole workgroup; the caller
// synchronizes afterwards).
__device__ __forceinline__ void fill_stream_table(const int4* tiles, const int* rows_tok, int* table,
                                                  const SSched& sc,
                                                  int base, int nwg, int ngrp, int BPI, int k0,
                                                  int cnt) {
    for (int i = threadIdx.x; i < cnt * kSTabInts; i += blockDim.x) {
        const int k = i / kSTabInts, f = i % kSTabInts;
        const int4 un = s_unit(sc, base, nwg, BPI, k0 + k);
        const int4 tile = tiles[un.x / ngrp];
        int v;
        if (f == 0) v = tile.x;
        else if (f == 1) v = tile.y;
        else if (f == 2) v = tile.z;
        else if (f == 3) v = un.x % ngrp;
        else if (f < 20) {
            const int row = f - 4;
            v = rows_tok ? rows_tok[tile.y + (row < tile.z ? row : 0)] : 0;
        } else if (f == 20) v = un.y;
        else if (f == 21) v = un.z;
        else if (f == 22) v = un.w;
        else v = 0;
        table[i] = v;
    }
}

// Fused routing bounds: n <= kFusedRouteMax tokens of topk <= 8 slots plus a
// shared row each; with kTileRows-row tiles every expert then has one tile.
constexpr int kRtMaxRows = kFusedRouteMax * 8 + kFusedRouteMax;
constexpr int kRtMaxTiles = kFusedRouteMax * 8 + 1;
static_assert(kFusedRouteMax <= kTileRows, "one tile per expert");

// Selection and dispatch of a small batch by one 512-thread workgroup (all
// threads call it): wave t selects token t (topk_wave_nj, the router's own
// selection) into sids; dispatch_small then writes the tile list, tile
// counts and sorted token ids to tiles / nt / tok (LDS). The lead workgroup
// also stores the ids, weights and every dispatch output to the global
// buffers of r.disp. scratch: kSmallDispIds + 2 * (kDispMaxE + 2) ints of LDS.
template <int NJ>
__device__ __forceinline__ void fused_route(const FusedRoute r, int E, bool lead, int4* tiles, int* nt,
                                            int* tok, int* scratch) {
    int* sids = scratch;                       // n * topk ids
    int* hist = sids + kSmallDispIds;
    int* pre = hist + kDispMaxE + 2;
    const int wave = threadIdx.x >> 6;
    if (wave < r.n) {
        const int t = wave;
        topk_wave_nj<false, NJ>(nullptr, nullptr, E, r.topk, r.norm_topk, r.routed_scale,
                                lead ? r.ids + t * r.topk : nullptr,
                                lead ? r.w + t * r.topk : nullptr, nullptr,
                                r.cs + (size_t)t * E,
                                reinterpret_cast<const float*>(r.cs) + (size_t)r.n * E + (size_t)t * E,
                                sids + t * r.topk);
    }
    __syncthreads();
    if (r.n == 1) {
        // One token: its topk ids are distinct experts, one row each, so an
        // expert's offset and tile index are its rank among the ids (the
        // outputs dispatch_small gives, without its histogram and scan).
        const int K = r.topk, sh = r.disp.with_shared;
        const int t = threadIdx.x;
        if (t < K) {
            const int e = sids[t];
            int rank = 0;
            for (int k = 0; k < K; ++k) rank += sids[k] < e ? 1 : 0;
            tiles[rank] = make_int4(e, rank, 1, 1 << 16);
            tok[rank] = 0;
            if (lead) {
                r.disp.tiles[rank] = make_int4(e, rank, 1, 1 << 16);
                r.disp.sorted_tok[rank] = 0;
                r.disp.sorted_slot[rank] = t;
                r.disp.inv[t] = rank;
            }
        } else if (t == K) {
            if (sh) {
                tiles[K] = make_int4(E, K, 1, 1 << 16);
                tok[K] = 0;
            }
            nt[0] = nt[1] = nt[2] = K + sh;
            if (lead) {
                if (sh) {
                    r.disp.tiles[K] = make_int4(E, K, 1, 1 << 16);
                    r.disp.sorted_tok[K] = 0;
                    r.disp.sorted_slot[K] = -1;
                }
                r.disp.ntiles[0] = r.disp.ntiles[1] = r.disp.ntiles[2] = K + sh;
                r.disp.offsets[E + 1] = K + sh;
            }
        }
        if (lead)
            for (int e = t; e <= E; e += 512) {
                int below = 0;
                for (int k = 0; k < K; ++k) below += sids[k] < e ? 1 : 0;
                r.disp.offsets[e] = below;
            }
        return;
    }
    dispatch_small<512>(sids, r.n, r.topk, E, r.disp.with_shared, tiles, nt, tok, r.disp, lead, hist,
                        pre);
}

template <int NMAT>
struct SLay {
    static constexpr int kRowB = kSGB * 256;                 // one row's 16 groups
    static constexpr int kXBytes = kTileRows * kRowB;        // 64 KiB
    static constexpr int kGOff = kXBytes;                    // X [16 groups][16 rows] fp32
    static constexpr int kBuf = kXBytes + kSGB * kTileRows * 4;
    static constexpr int kJunk = 2 * kBuf;                   // placeholder DMA target
    static constexpr int kRed = kJunk + 256;                 // [8][16] h group-sum partials
    static constexpr int kTab = kRed + 8 * 16 * 4;
    // Fused routing: the tile list, tile counts and sorted token ids the
    // kernel then reads in place of the global ones.
    static constexpr int kRtTiles = kTab + kTable * kSTabInts * 4;
    static constexpr int kRtNt = kRtTiles + kRtMaxTiles * 16;
    static constexpr int kRtTok = kRtNt + 16;
    static constexpr int kTotal = kRtTok + kRtMaxRows * 4;
    static_assert(kTotal <= 160 * 1024, "one workgroup's LDS");
    static constexpr int P = NMAT == 2 ? kSPGU : kSPDown;    // weight groups in flight per wave
    static_assert(kSGB % P == 0, "ring slots stay static across batches");
    static constexpr int kWL = 2 * NMAT;                     // loads per weight group
};

// NT: a non-temporal load (data read once: it does not displace the
// activation rows the workgroups re-read from L2).
template <bool NT>
__device__ __forceinline__ void gload16(u32x4& d, const void* base, uint32_t voff) {
    if constexpr (NT)
        asm volatile("global_load_dwordx4 %0, %1, %2 nt" : "=&v"(d) : "v"(voff), "s"(base));
    else
        asm volatile("global_load_dwordx4 %0, %1, %2" : "=&v"(d) : "v"(voff), "s"(base));
}
__device__ __forceinline__ void gload8(u32x2& d, const void* base, uint32_t voff) {
    asm volatile("global_load_dwordx2 %0, %1, %2" : "=&v"(d) : "v"(voff), "s"(base));
}

// Wave-uniform weight / scale bases of this wave's 16-row block in an item.
struct SWItem {
    const uint4* wq[2];
    const uint16_t* ws[2];
    int ng;   // weight groups of the unit
};

// PAIR (second projection): stream m is row block 16 g + 8 m + wave of the one
// matrix instead of block 8 g + wave of matrix m.
template <int NMAT, bool PAIR>
__device__ __forceinline__ SWItem sw_item(const ExpArgs& a, const int* table, int k, int wave,
                                          int nfb, int KG) {
    const uint4 h = lds_bcast16(lds_addr(table + k * kSTabInts));
    const uint4 u = lds_bcast16(lds_addr(table + k * kSTabInts + 20));
    const int e = sgpr(h.x);
    const int fb0 = sgpr(h.w) * (PAIR ? 16 : 8) + wave;
    const int g0 = sgpr(u.x) * kSGB;
    const bool sh = e == a.E;
    const size_t mstride_q = (size_t)nfb * KG * 64;
    const size_t mstride_s = (size_t)nfb * KG * 16;
    SWItem it;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const int mm = PAIR ? 0 : (m < NMAT ? m : 0);
        const int fb = PAIR ? fb0 + 8 * m : fb0;
        it.wq[m] = (sh ? a.swq[mm] : a.wq[mm] + (size_t)e * mstride_q) + ((size_t)fb * KG + g0) * 64;
        it.ws[m] = (sh ? a.sws[mm] : a.ws[mm] + (size_t)e * mstride_s) + ((size_t)fb * KG + g0) * 16;
    }
    it.ng = sgpr(u.y) * kSGB;
    return it;
}

// Activation-stream sources of one item: the src rows of this wave's two
// staged rows (2 wave, 2 wave + 1) and of this lane's group-sum row.
struct SAItem {
    uint32_t tok[2];
    uint32_t live[2];   // this wave's staged rows lie inside the tile (row < nrows)
    uint32_t gtok;
    int kb0, nb;        // the unit's batches
};

// GATHER (first projection): src rows are the tile's token ids; else the
// tile's own rows r0 + row.
template <bool GATHER>
__device__ __forceinline__ SAItem sa_item(const int* table, int k, int wave, int lane) {
    const uint32_t base = lds_addr(table + k * kSTabInts);
    const uint4 h = lds_bcast16(base);
    const uint4 u = lds_bcast16(base + 80);
    const int r0 = sgpr(h.y), nr = sgpr(h.z);
    SAItem it;
    it.kb0 = sgpr(u.x);
    it.nb = sgpr(u.y);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int row = 2 * wave + j;
        it.tok[j] = GATHER ? (uint32_t)sgpr(lds_read_u32(base + 16 + row * 4))
                              : (uint32_t)(r0 + (row < nr ? row : 0));
        it.live[j] = row < nr ? 1u : 0u;
    }
    const int row = lane & 15;
    it.gtok = GATHER ? lds_read_u32(base + 16 + row * 4) : (uint32_t)(r0 + (row < nr ? row : 0));
    return it;
}

// Exactly kSActDma DMAs per wave: activation batch bi (K-groups 16 bi ..) of an
// item into buffer `buf`. Row r of the batch sits at r * kRowB; chunk c of
// group j at j * 256 + 16 (c ^ (r & 15)).
template <int NMAT>
__device__ __forceinline__ void s_issue_act(const ExpArgs& a, const SAItem& it, int bi, int K,
                                            int KG, char* buf, char* junk, int wave, int lane) {
    using LY = SLay<NMAT>;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int j = m >> 2, quarter = m & 3;
        const int row = 2 * wave + j;
        const int grp = bi * kSGB + quarter * 4 + (lane >> 4);
        const int c = (lane & 15) ^ (row & 15);
        // Rows past the tile's end feed MFMA columns that are never stored:
        // every lane then fetches the same 16 bytes (one cache line per
        // instruction) instead of a duplicate row.
        const int off = it.live[j] ? grp * 128 + c * 8 : 0;
        dma16(a.src + (size_t)it.tok[j] * K + off, buf + row * LY::kRowB + quarter * 1024);
    }
    // Group sums: waves 0-3, lane l -> entry 64 wave + l = group 4 wave + l / 16, row l % 16.
    const int grp = bi * kSGB + ((wave & 3) * 4 + (lane >> 4));
    dma4(a.gsum + (size_t)it.gtok * KG + grp, wave < 4 ? buf + LY::kGOff + wave * 256 : junk);
}

template <int NMAT, bool NT>
__device__ __forceinline__ void s_issue_w(const SWItem& it, int kg, int lane, u32x4 (&w)[2],
                                          u32x2 (&sc)[2]) {
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
        gload16<NT>(w[m], reinterpret_cast<const char*>(it.wq[m]) + kg * 1024, (uint32_t)(lane * 16));
        gload8(sc[m], reinterpret_cast<const char*>(it.ws[m]) + kg * 32, (uint32_t)((lane >> 4) * 8));
    }
}

template <int NMAT, int N>
__device__ __forceinline__ void s_wait_w(u32x4 (&w)[2], u32x2 (&sc)[2]) {
    if constexpr (NMAT == 2)
        asm volatile("s_waitcnt vmcnt(%c4)" : "+v"(w[0]), "+v"(w[1]), "+v"(sc[0]), "+v"(sc[1]) : "i"(N));
    else
        asm volatile("s_waitcnt vmcnt(%c2)" : "+v"(w[0]), "+v"(sc[0]) : "i"(N));
}

// LDS operands of group j of a batch: the 4 activation fragments and X.
struct SOps {
    u32x4 x[4];
    float g;
};

// Per-lane LDS read bases of one activation buffer: fragment d of group j is
// at x[d] + 256 j, X of group j at g + 64 j (both immediate offsets).
struct SBase {
    uint32_t x[4];
    uint32_t g;
};

template <int NMAT>
__device__ __forceinline__ SBase s_base(const char* buf, int lane) {
    using LY = SLay<NMAT>;
    const int r = lane & 15, q = lane >> 4;
    SBase b;
#pragma unroll
    for (int d = 0; d < 4; ++d)
        b.x[d] = lds_addr(buf) + (uint32_t)(r * LY::kRowB + (((4 * q + d) ^ r) * 16));
    b.g = lds_addr(buf + LY::kGOff) + (uint32_t)(r * 4);
    return b;
}

template <int J>
__device__ __forceinline__ void s_load_ops(const SBase& b, SOps& o) {
#pragma unroll
    for (int d = 0; d < 4; ++d)
        asm volatile("ds_read_b128 %0, %1 offset:%c2" : "=&v"(o.x[d]) : "v"(b.x[d]), "i"(J * 256));
    asm volatile("ds_read_b32 %0, %1 offset:%c2" : "=&v"(o.g) : "v"(b.g), "i"(J * 64));
}

__device__ __forceinline__ void s_wait_ops(SOps& o) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(o.x[0]), "+v"(o.x[1]), "+v"(o.x[2]), "+v"(o.x[3]), "+v"(o.g));
}

template <int NMAT>
__device__ __forceinline__ void s_compute(const SOps& o, const u32x4 (&w)[2], const u32x2 (&sc)[2],
                                          const DqConst& dqc, f32x4 (&acc)[NMAT]) {
    const float off = -136.0f * o.g;
    f32x4 p[NMAT];
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
            p[m] = mfma16x16x32(dq_w4(w[m][d], dqc), as_bf16x8(o.x[d]),
                                d == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : p[m]);
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
        const float s4[4] = {bf16_to_f32(sc[m].x & 0xffffu), __uint_as_float(sc[m].x & 0xffff0000u),
                             bf16_to_f32(sc[m].y & 0xffffu), __uint_as_float(sc[m].y & 0xffff0000u)};
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc[m][jj] = __builtin_fmaf(s4[jj], p[m][jj] + off, acc[m][jj]);
    }
}

// MODE 0: gate/up (two matrices, SiLU epilogue). MODE 2: down, two 16-row
// blocks per wave (a 256-row item), the same two-stream shape as gate/up,
// which halves the batches, barriers and item switches per weight byte
// against one block per wave (MODE 1, kept for shapes the layer does not
// pass).
template <int MODE, bool NTW>
__global__ __launch_bounds__(512) void w4_stream_kernel(ExpArgs a) {
    constexpr int NMAT = MODE == 1 ? 1 : 2;
    constexpr bool GU = MODE == 0, PAIR = MODE == 2;
    using LY = SLay<NMAT>;
    constexpr int P = LY::P;
    extern __shared__ __align__(16) char lds[];
    const int4* tiles = a.tiles;
    const int* ntiles = a.ntiles;
    const int* rows_tok = a.rows_tok;
    static_assert((kSmallDispIds + 2 * (kDispMaxE + 2)) * 4 <= LY::kBuf, "fused routing scratch inside activation buffer 1");
    static_assert(kFusedRouteMax * 8 <= kSmallDispIds, "the small dispatch holds every id");
    if constexpr (GU) {
        if (a.route.cs) {
            // Select and dispatch here; the tile list then lives in LDS. The
            // dispatch scratch sits in activation buffer 1, unused until the
            // first batch is under way.
            int4* tl = reinterpret_cast<int4*>(lds + LY::kRtTiles);
            int* nt = reinterpret_cast<int*>(lds + LY::kRtNt);
            int* tok = reinterpret_cast<int*>(lds + LY::kRtTok);
            int* scr = reinterpret_cast<int*>(lds + LY::kBuf);
            // The lead is the last workgroup: the one with the least expert
            // work, which hides the wait for its global stores.
            const bool lead = blockIdx.x == gridDim.x - 1;
            const int E = a.E;
            if (E <= 64) fused_route<1>(a.route, E, lead, tl, nt, tok, scr);
            else if (E <= 128) fused_route<2>(a.route, E, lead, tl, nt, tok, scr);
            else if (E <= 256) fused_route<4>(a.route, E, lead, tl, nt, tok, scr);
            else fused_route<8>(a.route, E, lead, tl, nt, tok, scr);
            tiles = tl;
            ntiles = nt;
            rows_tok = tok;
            __syncthreads();
        }
    }
    const DqConst dqc = dq_const();
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;
    const int K = GU ? a.H : a.I;
    const int KG = K / 128;
    const int BPI = KG / kSGB;                 // activation batches per item
    const int nfb = (GU ? a.I : a.H) / 16;
    const int ngrp = nfb / (PAIR ? 16 : 8);
    const int total = sgpr(*ntiles) * ngrp;   // uniform (ntiles may point into LDS)
    const int nwg = (int)gridDim.x;
    const int base = (int)blockIdx.x;
    const SSched sch = s_sched(total, nwg, base, GU ? BPI : 1, a.tcap);
    const int nitems = sch.nunits;
    int* table = reinterpret_cast<int*>(lds + LY::kTab);
    char* junk = lds + LY::kJunk;

    // Finishes an item from its total T: h = silu(gate) * up as bf16 and the
    // group sum of the rounded h per tile row (gate/up), or the fp32 partial
    // row (down).
    auto finish = [&](const f32x4 (&T)[NMAT], int r0, int nr, int fb) {
        const bool valid = r < nr;
        const size_t row = (size_t)r0 + r;
        if constexpr (GU) {
            const uint32_t h01 = pack_bf16x2(silu_fast(T[0][0]) * T[1][0],
                                             silu_fast(T[0][1]) * T[1][1]);
            const uint32_t h23 = pack_bf16x2(silu_fast(T[0][2]) * T[1][2],
                                             silu_fast(T[0][3]) * T[1][3]);
            if (valid)
                *reinterpret_cast<uint2*>(a.h + row * a.I + fb * 16 + 4 * q) = uint2{h01, h23};
            float ps = (bf16_to_f32(h01 & 0xffffu) + __uint_as_float(h01 & 0xffff0000u)) +
                       (bf16_to_f32(h23 & 0xffffu) + __uint_as_float(h23 & 0xffff0000u));
            ps = ps + __shfl_xor(ps, 16);
            ps = ps + __shfl_xor(ps, 32);
            const uint32_t red = lds_addr(lds + LY::kRed);
            if (q == 0) lds_write_f32(red + (uint32_t)((wave * 16 + r) * 4), ps);
            __builtin_amdgcn_s_barrier();
            if (wave == 0 && q == 0) {
                float tot = 0.0f;
#pragma unroll
                for (int w = 0; w < 8; ++w)
                    tot += __uint_as_float(lds_read_u32(red + (uint32_t)((w * 16 + r) * 4)));
                if (valid) a.hsum[row * (a.I / 128) + fb / 8] = tot;
            }
            __builtin_amdgcn_s_barrier();
        } else {
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
                if (valid)
                    *reinterpret_cast<float4*>(a.dpart + row * a.H + (fb + 8 * m) * 16 + 4 * q) =
                        make_float4(T[m][0], T[m][1], T[m][2], T[m][3]);
        }
    };

    for (int k0 = 0; k0 < nitems; k0 += kTable) {
        const int cnt = min(kTable, nitems - k0);
        fill_stream_table(tiles, rows_tok, table, sch, base, nwg, ngrp, GU ? BPI : 1, k0, cnt);
        __syncthreads();
        // Activation batches of the chunk: whole items BPI each, parts 1.
        const int nwhole = sch.split ? max(0, min(cnt, sch.R - k0)) : cnt;
        const int nbatch = nwhole * BPI + (cnt - nwhole);

        // Weight stream, P groups ahead (crosses items).
        int wk = 0, wkg = 0;
        SWItem wit = sw_item<NMAT, PAIR>(a, table, 0, wave, nfb, KG);
        u32x4 W[P][2];
        u32x2 Sc[P][2];
        // Past the chunk's last group both streams re-issue their final
        // loads, so every step issues the same loads and all waits stay
        // static; the surplus data is never read.
        auto issue_w = [&](u32x4 (&w)[2], u32x2 (&sc)[2]) {
            s_issue_w<NMAT, NTW>(wit, wkg, lane, w, sc);
            if (wkg + 1 < wit.ng) {
                ++wkg;
            } else if (wk + 1 < cnt) {
                ++wk;
                wkg = 0;
                wit = sw_item<NMAT, PAIR>(a, table, wk, wave, nfb, KG);
            }
        };
        // Activation stream, one batch ahead.
        int ak = 0, abi = 0;
        SAItem ait = sa_item<GU>(table, 0, wave, lane);
        auto issue_act = [&](int b) {
            s_issue_act<NMAT>(a, ait, ait.kb0 + abi, K, KG, lds + (b & 1) * LY::kBuf, junk, wave,
                              lane);
            if (abi + 1 < ait.nb) {
                ++abi;
            } else if (ak + 1 < cnt) {
                ++ak;
                abi = 0;
                ait = sa_item<GU>(table, ak, wave, lane);
            }
        };

        issue_act(0);
#pragma unroll
        for (int i = 0; i < P; ++i) issue_w(W[i], Sc[i]);
        wait_vmcnt<P * LY::kWL>();
        __builtin_amdgcn_s_barrier();
        SOps ops[2];
        s_load_ops<0>(s_base<NMAT>(lds, lane), ops[0]);

        int cur_k = 0, cur_bi = 0;
        int cr0 = 0, cnr = 0, cfb = 0, ckb = 0, cnb = 0, ctail = -1;
        auto load_cur = [&]() {
            const uint4 h = lds_bcast16(lds_addr(table + cur_k * kSTabInts));
            const uint4 u = lds_bcast16(lds_addr(table + cur_k * kSTabInts + 20));
            cr0 = sgpr(h.y); cnr = sgpr(h.z); cfb = sgpr(h.w) * (PAIR ? 16 : 8) + wave;
            ckb = sgpr(u.x); cnb = sgpr(u.y); ctail = sgpr(u.z);
        };
        load_cur();
        f32x4 acc[NMAT], T[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) acc[m] = T[m] = f32x4{0.f, 0.f, 0.f, 0.f};

        for (int B = 0; B < nbatch; ++B) {
            const bool next_act = B + 1 < nbatch;
            const SBase cb = s_base<NMAT>(lds + (B & 1) * LY::kBuf, lane);
            static_for<kSGB>([&](auto jc) {
                constexpr int j = decltype(jc)::value;
                if constexpr (j == 8) issue_act(B + 1);
                // Weights of group j: loads issued after them are the groups
                // j + 1 .. j + P - 1 and, for 8 <= j < 8 + P, batch B + 1.
                if constexpr (j >= 8 && j < 8 + P)
                    s_wait_w<NMAT, (P - 1) * LY::kWL + kSActDma>(W[j % P], Sc[j % P]);
                else
                    s_wait_w<NMAT, (P - 1) * LY::kWL>(W[j % P], Sc[j % P]);
                SOps& o = ops[j & 1];
                s_wait_ops(o);
                if constexpr (j + 1 < kSGB) s_load_ops<j + 1>(cb, ops[(j + 1) & 1]);
                s_compute<NMAT>(o, W[j % P], Sc[j % P], dqc, acc);
                // Pin the rescale to this step (otherwise it is deferred and
                // every step's partial products and scales stay live).
#pragma unroll
                for (int m = 0; m < NMAT; ++m) asm volatile("" : "+v"(acc[m]));
                // The slot is free again: group j + P goes into it.
                issue_w(W[j % P], Sc[j % P]);
                __builtin_amdgcn_sched_barrier(0);
            });
            // Batch total into the unit's running total, batch order.
#pragma unroll
            for (int m = 0; m < NMAT; ++m) {
                T[m] = cur_bi == 0 ? acc[m] : T[m] + acc[m];
                acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
            if (++cur_bi == cnb) {
                if (ctail < 0) {
                    finish(T, cr0, cnr, cfb);
                } else {
                    // A part: store t_b; the item is finished after the ticket.
                    // [value][thread]: each store instruction covers 256
                    // contiguous bytes (whole lines).
                    float* dst = a.tpart + (size_t)(ctail * BPI + ckb) * 4096 + threadIdx.x;
#pragma unroll
                    for (int m = 0; m < NMAT; ++m)
#pragma unroll
                        for (int i = 0; i < 4; ++i) st_dev(dst + (m * 4 + i) * 512, T[m][i]);
                }
                cur_bi = 0;
                if (++cur_k < cnt) load_cur();
            }
            if (next_act) {
                // Batch B + 1 has landed once only the 8 weight groups issued
                // after it (from j = 8 on) are pending.
                wait_vmcnt<8 * LY::kWL>();
                __builtin_amdgcn_s_barrier();
                s_load_ops<0>(s_base<NMAT>(lds + ((B + 1) & 1) * LY::kBuf, lane), ops[0]);
            }
        }
        wait_vmcnt<0>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
    }
    if constexpr (GU) {
        // Parts: every wave's stores have completed (vmcnt(0) above); the
        // workgroup with an item's last ticket finishes it.
        int* flag = reinterpret_cast<int*>(junk);
        for (int u = sch.split ? sch.R : nitems; u < nitems; ++u) {
            const int4 un = s_unit(sch, base, nwg, BPI, u);
            if (threadIdx.x == 0) {
                const bool last = ticket_dev(&a.tick[un.w]) == (unsigned)(BPI - 1);
                *flag = last ? 1 : 0;
            }
            __syncthreads();
            const bool last = *flag != 0;
            __syncthreads();
            if (!last) continue;
            f32x4 T[NMAT];
            for (int b = 0; b < BPI; ++b) {
                const float* src = a.tpart + (size_t)(un.w * BPI + b) * 4096 + threadIdx.x;
#pragma unroll
                for (int m = 0; m < NMAT; ++m) {
                    const f32x4 t{ld_dev(src + (m * 4) * 512), ld_dev(src + (m * 4 + 1) * 512),
                                  ld_dev(src + (m * 4 + 2) * 512), ld_dev(src + (m * 4 + 3) * 512)};
                    T[m] = b == 0 ? t : T[m] + t;
                }
            }
            const int4 tile = tiles[un.x / ngrp];
            finish(T, tile.y, tile.z, (un.x % ngrp) * 8 + wave);
        }
    }
}

template <int MODE>
static int launch_stream(const ExpArgs& a, long max_work, hipStream_t s, bool nt) {
    using LY = SLay<MODE == 1 ? 1 : 2>;
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&w4_stream_kernel<MODE, false>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, LY::kTotal) != hipSuccess ||
            hipFuncSetAttribute(reinterpret_cast<const void*>(&w4_stream_kernel<MODE, true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, LY::kTotal) != hipSuccess)
            return -4;
        attr_set = true;
    }
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    long blocks = max_work;
    if (blocks > (long)cus) blocks = cus;
    if (blocks < 1) blocks = 1;
    if (nt)
        hipLaunchKernelGGL((w4_stream_kernel<MODE, true>), dim3((unsigned)blocks), dim3(512), LY::kTotal, s, a);
    else
        hipLaunchKernelGGL((w4_stream_kernel<MODE, false>), dim3((unsigned)blocks), dim3(512), LY::kTotal, s,
                           a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// ---------------------------------------------------------------------------
// Combine: out[t] = (((0 + w0*y0) + w1*y1) + ...) + y_shared, slot order then
// shared (src/model_glm52.cpp:1133-1152). Gather, no atomics: deterministic.
// ---------------------------------------------------------------------------
template <bool BF16>
__device__ __forceinline__ float4 combine_row(const float* dpart, size_t row, int H, int f4) {
    if constexpr (BF16) {
        const uint2 v = reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(dpart) + row * H)[f4];
        return make_float4(bf16_to_f32(v.x & 0xffffu), __uint_as_float(v.x & 0xffff0000u),
                           bf16_to_f32(v.y & 0xffffu), __uint_as_float(v.y & 0xffff0000u));
    } else {
        return reinterpret_cast<const float4*>(dpart + row * H)[f4];
    }
}

// BF16: the partial rows are bf16 (large-group kernels), else fp32.
template <bool BF16>
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
        const float4 y = combine_row<BF16>(dpart, (size_t)inv[(size_t)t * topk + s], H, f4);
        acc.x = acc.x + ws * y.x; acc.y = acc.y + ws * y.y;
        acc.z = acc.z + ws * y.z; acc.w = acc.w + ws * y.w;
    }
    if (with_shared) {
        const float4 y = combine_row<BF16>(dpart, (size_t)n * topk + t, H, f4);
        acc.x = acc.x + y.x; acc.y = acc.y + y.y; acc.z = acc.z + y.z; acc.w = acc.w + y.w;
    }
    reinterpret_cast<float4*>(out + (size_t)t * H)[f4] = acc;
}

// The bf16 partial rows of the large-group kernels, topk <= 8: 8 features
// (16 B of each row) per thread, every row's load issued before the adds.
// The same per-element operations in the same order as combine_kernel.
__global__ __launch_bounds__(256) void combine_bf16x8_kernel(const uint16_t* __restrict__ dpart,
                                                             const int* __restrict__ inv,
                                                             const float* __restrict__ w, int n,
                                                             int topk, int H, int with_shared,
                                                             float* __restrict__ out) {
    const int t = blockIdx.y;
    const int f8 = blockIdx.x * blockDim.x + threadIdx.x;
    if (f8 * 8 >= H) return;
    uint4 v[9];
    float ws[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        if (s < topk) {
            ws[s] = w[(size_t)t * topk + s];
            v[s] = reinterpret_cast<const uint4*>(dpart + (size_t)inv[(size_t)t * topk + s] * H)[f8];
        }
    }
    if (with_shared) v[8] = reinterpret_cast<const uint4*>(dpart + ((size_t)n * topk + t) * H)[f8];
    auto el = [](const uint4& r, int q) {
        const uint32_t d = q < 2 ? r.x : q < 4 ? r.y : q < 6 ? r.z : r.w;
        return (q & 1) ? __uint_as_float(d & 0xffff0000u) : bf16_to_f32(d & 0xffffu);
    };
    float acc[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s)
        if (s < topk)
#pragma unroll
            for (int q = 0; q < 8; ++q) acc[q] = acc[q] + ws[s] * el(v[s], q);
    if (with_shared)
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[q] = acc[q] + el(v[8], q);
    float4* o = reinterpret_cast<float4*>(out + (size_t)t * H) + 2 * f8;
    o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
}

// The fp32 partial rows of the decode kernels, topk <= 8: 4 features (16 B
// of each row) per thread, the slots' indices and weights loaded first, then
// every row's 16 bytes, then the adds: combine_kernel's operations in its
// order, with two dependent load rounds instead of two per slot.
__global__ __launch_bounds__(256) void combine_f32x4_kernel(const float* __restrict__ dpart,
                                                            const int* __restrict__ inv,
                                                            const float* __restrict__ w, int n,
                                                            int topk, int H, int with_shared,
                                                            float* __restrict__ out) {
    const int t = blockIdx.y;
    const int f4 = blockIdx.x * blockDim.x + threadIdx.x;
    if (f4 * 4 >= H) return;
    int row[8];
    float ws[8];
#pragma unroll
    for (int s = 0; s < 8; ++s)
        if (s < topk) {
            row[s] = inv[(size_t)t * topk + s];
            ws[s] = w[(size_t)t * topk + s];
        }
    float4 y[9];
#pragma unroll
    for (int s = 0; s < 8; ++s)
        if (s < topk) y[s] = reinterpret_cast<const float4*>(dpart + (size_t)row[s] * H)[f4];
    if (with_shared) y[8] = reinterpret_cast<const float4*>(dpart + ((size_t)n * topk + t) * H)[f4];
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < 8; ++s)
        if (s < topk) {
            acc.x = acc.x + ws[s] * y[s].x; acc.y = acc.y + ws[s] * y[s].y;
            acc.z = acc.z + ws[s] * y[s].z; acc.w = acc.w + ws[s] * y[s].w;
        }
    if (with_shared) {
        acc.x = acc.x + y[8].x; acc.y = acc.y + y[8].y; acc.z = acc.z + y[8].z; acc.w = acc.w + y[8].w;
    }
    reinterpret_cast<float4*>(out + (size_t)t * H)[f4] = acc;
}

// ---------------------------------------------------------------------------
// Ring depth and batch size per projection (one 8-wave workgroup per CU).
constexpr int kRingGU = 3;
constexpr int kRingDown = 4;
constexpr int kPFGU = 2;
constexpr int kPFDown = 2;
constexpr int kNWGU = 8;
constexpr int kNWDown = 8;

template <int NMAT, int PF, int D, int NW>
static int launch_expert(const ExpArgs& a, long max_work, hipStream_t s) {
    using RG = Ring<NMAT, PF, D, NW>;
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&w4_expert_kernel<NMAT, PF, D, NW>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, RG::kTotal) !=
            hipSuccess)
            return -4;
        attr_set = true;
    }
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    // Persistent: 8 waves per CU, never more workgroups than items.
    long blocks = max_work;
    if (blocks > (long)cus * (8 / NW)) blocks = (long)cus * (8 / NW);
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL((w4_expert_kernel<NMAT, PF, D, NW>), dim3((unsigned)blocks), dim3(NW * 64),
                       RG::kTotal, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

bool fused_route_ok(int n, int topk, int E, int H) {
    return n >= 1 && n <= kFusedRouteMax && topk >= 1 && topk <= 8 && topk <= E && E <= kDispMaxE &&
           (H / 128) % kSGB == 0 && H % 128 == 0;
}

int launch_gate_up(const ExpertPtrs& P, const uint16_t* x, const float* xsum, const int* tiles,
                   const int* ntiles, int max_tiles, const int* rows_tok, uint16_t* h,
                   float* hsum, unsigned int* tick, float* tpart, size_t tpart_bytes, int H, int I,
                   int E, hipStream_t s, const FusedRoute* route, bool stream_weights) {
    ExpArgs a{};
    if (route) {
        if (!fused_route_ok(route->n, route->topk, E, H)) return -1;
        a.route = *route;
    }
    a.tick = tick; a.tpart = tpart;
    a.tcap = tick && tpart ? (int)(tpart_bytes / kTailPartBytes) : 0;
    a.wq[0] = reinterpret_cast<const uint4*>(P.gate_q); a.ws[0] = P.gate_s;
    a.wq[1] = reinterpret_cast<const uint4*>(P.up_q); a.ws[1] = P.up_s;
    a.swq[0] = reinterpret_cast<const uint4*>(P.sh_gate_q); a.sws[0] = P.sh_gate_s;
    a.swq[1] = reinterpret_cast<const uint4*>(P.sh_up_q); a.sws[1] = P.sh_up_s;
    a.src = x; a.gsum = xsum; a.tiles = reinterpret_cast<const int4*>(tiles); a.ntiles = ntiles;
    a.rows_tok = rows_tok; a.h = h; a.hsum = hsum; a.H = H; a.I = I; a.E = E;
    const long work = (long)max_tiles * (I / 16 / kNWGU);
    if ((H / 128) % kSGB == 0)
        return launch_stream<0>(a, (long)max_tiles * (I / 128) * (H / 128 / kSGB), s, stream_weights);
    if (route) return -1;
    if ((H / 128) % kPFGU == 0) return launch_expert<2, kPFGU, kRingGU, kNWGU>(a, work, s);
    return launch_expert<2, 1, 6, kNWGU>(a, work, s);   // odd K-group count
}

int launch_down(const ExpertPtrs& P, const uint16_t* h, const float* hsum, const int* tiles,
                const int* ntiles, int max_tiles, float* dpart, int H, int I, int E,
                hipStream_t s, bool stream_weights) {
    ExpArgs a{};
    a.wq[0] = reinterpret_cast<const uint4*>(P.down_q); a.ws[0] = P.down_s;
    a.swq[0] = reinterpret_cast<const uint4*>(P.sh_down_q); a.sws[0] = P.sh_down_s;
    a.wq[1] = a.wq[0]; a.ws[1] = a.ws[0]; a.swq[1] = a.swq[0]; a.sws[1] = a.sws[0];
    a.src = h; a.gsum = hsum; a.tiles = reinterpret_cast<const int4*>(tiles); a.ntiles = ntiles;
    a.dpart = dpart; a.H = H; a.I = I; a.E = E;
    const long work = (long)max_tiles * (H / 16 / kNWDown);
    // Two 16-row blocks per wave (the layer's hidden size is a multiple of 256).
    if ((I / 128) % kSGB == 0 && H % 256 == 0) return launch_stream<2>(a, (long)max_tiles * (H / 256), s, stream_weights);
    if ((I / 128) % kPFDown == 0) return launch_expert<1, kPFDown, kRingDown, kNWDown>(a, work, s);
    return launch_expert<1, 1, 6, kNWDown>(a, work, s);   // odd K-group count
}

int launch_combine(const float* dpart, const int* inv, const float* w, int n, int topk, int H,
                   int with_shared, float* out, hipStream_t s, bool bf16) {
    if (bf16 && topk <= 8 && H % 8 == 0) {
        hipLaunchKernelGGL(combine_bf16x8_kernel, dim3((unsigned)((H / 8 + 255) / 256), (unsigned)n),
                           dim3(256), 0, s, reinterpret_cast<const uint16_t*>(dpart), inv, w, n, topk,
                           H, with_shared, out);
        return hipGetLastError() == hipSuccess ? 0 : -4;
    }
    dim3 grid((unsigned)((H / 4 + 255) / 256), (unsigned)n);
    if (!bf16 && topk <= 8 && H % 4 == 0) {
        hipLaunchKernelGGL(combine_f32x4_kernel, grid, dim3(256), 0, s, dpart, inv, w, n, topk, H,
                           with_shared, out);
        return hipGetLastError() == hipSuccess ? 0 : -4;
    }
    if (bf16)
        hipLaunchKernelGGL(combine_kernel<true>, grid, dim3(256), 0, s, dpart, inv, w, n, topk, H,
                           with_shared, out);
    else
        hipLaunchKernelGGL(combine_kernel<false>, grid, dim3(256), 0, s, dpart, inv, w, n, topk,
                           H, with_shared, out);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace glmmoe
