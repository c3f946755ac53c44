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
// Streaming. Everything a batch of PF 128-K groups needs -- each wave's
// weight tiles and scales, and the tile's 16 activation rows (shared by the
// workgroup's 4 waves, which always work on the same tile) -- is copied
// global -> LDS by the LDS-DMA path (global_load_lds_dwordx4 / _dword), so
// nothing in flight occupies registers. A ring of D batch slots keeps D-1
// batches in flight per wave. Every wave issues the same number of DMA
// instructions per batch (kDma), so "batch b has landed" is the immediate
// s_waitcnt vmcnt(kDma * (D - 2)); one s_barrier per batch then publishes the
// shared rows and frees the oldest slot. The pipeline runs across work items
// (a wave's items are w0, w0 + nwaves, ...), so it never drains between
// them. LDS reads are inline ds_read_b128 with their own lgkmcnt wait, which
// keeps the compiler from inserting a vmcnt(0) for the pending DMA. Their
// outputs are early-clobber: a read returns asynchronously, so no output may
// share a register with an address still needed by a later read.
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
    const int4* tiles; const int* ntiles; const int* rows_tok;
    uint16_t* h; float* dpart;
    int H, I, E;
};

template <int NMAT, int PF, int D>
struct Ring {
    static_assert(PF == 2 || PF == 4, "a batch row span is 512 or 1024 bytes");
    static constexpr int kW = 1024;                           // one weight tile
    static constexpr int kWBytes = 4 * NMAT * PF * kW;        // all waves' tiles
    static constexpr int kSBytes = 4 * 256;                   // scale dwords per wave
    static constexpr int kSpan = PF * 256;                    // bytes of one row per batch
    static constexpr int kRPI = 1024 / kSpan;                 // rows per 1 KiB DMA
    static constexpr int kPair = 1024 + 16 * kRPI;            // padded stride of one DMA
    static constexpr int kXBytes = (16 / kRPI) * kPair;
    static constexpr int kSlot = kWBytes + kSBytes + kXBytes;
    static constexpr int kBytes = D * kSlot;
    static constexpr int kTotal = kBytes + kTable * kTabInts * 4;   // + the item table
    static_assert(2 * kTotal <= 160 * 1024, "two workgroups per CU");
    static constexpr int kXDma = 4 / kRPI;                    // activation DMAs per wave
    static constexpr int kDma = NMAT * PF + 1 + kXDma;        // DMA instructions per batch per wave
    // Byte offset of chunk 0 of activation row r inside the slot's activation
    // area. A DMA block holds kRPI rows interleaved at 16 B (chunk c of row r
    // at block(r / kRPI) + 16 kRPI c + 16 (r % kRPI)); with the block stride
    // kPair, the 16 rows an MFMA fragment reads fall on distinct banks.
    static __device__ __forceinline__ int row_off(int r) { return (r / kRPI) * kPair + (r % kRPI) * 16; }
    static constexpr int kChunk = 16 * kRPI;                  // stride between a row's chunks
};

// Work items of a workgroup come in steps k: the 4 waves take items
// base + wave + k * nwaves, which share one tile. A chunk of up to kTable
// steps is described in an LDS table read back with inline ds_read (no
// vector-memory loads inside the pipeline, whose waits would drain the DMA
// queue): per step {expert, row0, nrows, feature block of wave 0} and the 16
// token ids of the tile rows (row 0's token past nrows).

struct Item {
    const uint4* wq[2];
    const uint16_t* ws[2];
    int r0, nr, fb;
    int tok[4];   // tokens (NMAT = 2) or grouped rows (NMAT = 1) of this wave's 4 staged rows
};

template <int NMAT>
__device__ __forceinline__ Item item_from_table(const ExpArgs& a, const int* table, int k,
                                                int wave, int nfb, int KG) {
    const uint32_t base = lds_addr(table + k * kTabInts);
    const uint4 h = lds_bcast16(base);
    const uint4 t = lds_bcast16(base + 16 + wave * 16);
    Item it;
    const int e = sgpr(h.x);
    it.r0 = sgpr(h.y);
    it.nr = sgpr(h.z);
    it.fb = sgpr(h.w) + wave;
    if (NMAT == 2) {
        it.tok[0] = sgpr(t.x); it.tok[1] = sgpr(t.y); it.tok[2] = sgpr(t.z); it.tok[3] = sgpr(t.w);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = wave * 4 + j;
            it.tok[j] = it.r0 + (row < it.nr ? row : 0);
        }
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
__device__ __forceinline__ void fill_table(const ExpArgs& a, int* table, long base, long nwaves,
                                           int nfb, long k0, int cnt) {
    for (int i = threadIdx.x; i < cnt * kTabInts; i += blockDim.x) {
        const int k = i / kTabInts, f = i % kTabInts;
        const long item = base + (k0 + k) * nwaves;
        const int4 tile = a.tiles[item / nfb];
        int v;
        if (f == 0) v = tile.x;
        else if (f == 1) v = tile.y;
        else if (f == 2) v = tile.z;
        else if (f == 3) v = (int)(item % nfb);
        else {
            const int row = f - 4;
            v = a.rows_tok ? a.rows_tok[tile.y + (row < tile.z ? row : 0)] : 0;
        }
        table[i] = v;
    }
}

// Issues batch bb of item `it` into ring slot `slot` (exactly kDma DMAs).
template <int NMAT, int PF, int D>
__device__ __forceinline__ void issue_batch(const ExpArgs& a, const Item& it, int bb, int K,
                                            int KG, char* slot, int wave, int lane) {
    using RG = Ring<NMAT, PF, D>;
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
    // Activation rows 4*wave .. 4*wave+3 of the tile, kRPI rows per DMA (row r0
    // stands in past nr; those token columns are computed but never stored).
#pragma unroll
    for (int j = 0; j < RG::kXDma; ++j) {
        const int sub = lane % RG::kRPI;                 // row inside this DMA
        const int li = lane / RG::kRPI;                  // 16-byte chunk inside the row
        const int jr = j * RG::kRPI + sub;               // 0..3: which of this wave's rows
        size_t srow = (size_t)it.tok[0];
#pragma unroll
        for (int t = 1; t < 4; ++t) srow = jr == t ? (size_t)it.tok[t] : srow;
        const int koff = min(kg0 * 128 + li * 8, K - 8);  // bf16 offset of this lane's 16 B
        const int row0 = wave * 4 + j * RG::kRPI;         // first row of this DMA
        dma16(a.src + srow * K + koff,
              slot + RG::kWBytes + RG::kSBytes + (row0 / RG::kRPI) * RG::kPair);
    }
}

template <int NMAT, int PF, int D>
__device__ __forceinline__ void compute_batch(const char* slot, int bb, int KG, int wave,
                                              int lane, const DqConst& dqc, f32x4 (&acc)[NMAT]) {
    using RG = Ring<NMAT, PF, D>;
    const int r = lane & 15, q = lane >> 4;
    const uint32_t wbase = lds_addr(slot) + (uint32_t)(wave * NMAT * PF * RG::kW + lane * 16);
    const uint32_t sbase = lds_addr(slot + RG::kWBytes + wave * 256) + (uint32_t)(q * 8);
    const uint32_t xbase =
        lds_addr(slot + RG::kWBytes + RG::kSBytes) + (uint32_t)(RG::row_off(r) + 4 * q * RG::kChunk);
    // bf16 1.0 in every element: the A operand of the group-sum MFMA.
    const bf16x8 ones = __builtin_bit_cast(bf16x8, uint4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
#pragma unroll
    for (int i = 0; i < PF; ++i) {
        const bool live = bb * PF + i < KG;
        uint4 x0, x1, x2, x3, w0, w1;
        uint2 s0, s1;
        const uint32_t xa = xbase + i * 16 * RG::kChunk;   // group i = chunks 16i ..
        const uint32_t wa = wbase + i * RG::kW;
        const uint32_t sa = sbase + i * 32;
        if constexpr (NMAT == 2) {
            asm volatile(
                "ds_read_b128 %0, %8\n"
                "ds_read_b128 %1, %8 offset:%c13\n"
                "ds_read_b128 %2, %8 offset:%c14\n"
                "ds_read_b128 %3, %8 offset:%c15\n"
                "ds_read_b128 %4, %9\n"
                "ds_read_b128 %5, %9 offset:%c11\n"
                "ds_read_b64 %6, %10\n"
                "ds_read_b64 %7, %10 offset:%c12\n"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3), "=&v"(w0), "=&v"(w1), "=&v"(s0),
                  "=&v"(s1)
                : "v"(xa), "v"(wa), "v"(sa), "i"(PF * RG::kW), "i"(PF * 32), "i"(RG::kChunk),
                  "i"(2 * RG::kChunk), "i"(3 * RG::kChunk));
        } else {
            asm volatile(
                "ds_read_b128 %0, %6\n"
                "ds_read_b128 %1, %6 offset:%c9\n"
                "ds_read_b128 %2, %6 offset:%c10\n"
                "ds_read_b128 %3, %6 offset:%c11\n"
                "ds_read_b128 %4, %7\n"
                "ds_read_b64 %5, %8\n"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3), "=&v"(w0), "=&v"(s0)
                : "v"(xa), "v"(wa), "v"(sa), "i"(RG::kChunk), "i"(2 * RG::kChunk),
                  "i"(3 * RG::kChunk));
            w1 = w0;
            s1 = s0;
        }
        f32x4 px = {0.f, 0.f, 0.f, 0.f};
        px = mfma16x16x32(ones, as_bf16x8(x0), px);
        px = mfma16x16x32(ones, as_bf16x8(x1), px);
        px = mfma16x16x32(ones, as_bf16x8(x2), px);
        px = mfma16x16x32(ones, as_bf16x8(x3), px);
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            const uint4 wv = m == 0 ? w0 : w1;
            const uint2 sv = m == 0 ? s0 : s1;
            float sc[4];
            sc[0] = bf16_to_f32(sv.x & 0xffffu); sc[1] = bf16_to_f32(sv.x >> 16);
            sc[2] = bf16_to_f32(sv.y & 0xffffu); sc[3] = bf16_to_f32(sv.y >> 16);
            f32x4 p = {0.f, 0.f, 0.f, 0.f};
            p = mfma16x16x32(dq_w4(wv.x, dqc), as_bf16x8(x0), p);
            p = mfma16x16x32(dq_w4(wv.y, dqc), as_bf16x8(x1), p);
            p = mfma16x16x32(dq_w4(wv.z, dqc), as_bf16x8(x2), p);
            p = mfma16x16x32(dq_w4(wv.w, dqc), as_bf16x8(x3), p);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[m][j] = __builtin_fmaf(live ? sc[j] : 0.0f,
                                           __builtin_fmaf(-136.0f, px[j], p[j]), acc[m][j]);
        }
    }
}

template <int NMAT, int PF, int D>
__global__ __launch_bounds__(256) void w4_expert_kernel(ExpArgs a) {
    using RG = Ring<NMAT, PF, D>;
    extern __shared__ __align__(16) char ring[];
    const DqConst dqc = dq_const();
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;
    const int K = NMAT == 2 ? a.H : a.I;
    const int KG = K / 128;
    const int nfb = (NMAT == 2 ? a.I : a.H) / 16;
    const int nbatch = (KG + PF - 1) / PF;
    const long total = (long)(*a.ntiles) * nfb;
    const long nwaves = (long)gridDim.x * 4;
    const long base = (long)blockIdx.x * 4;
    // Steps of this workgroup (equal for its 4 waves: total and nwaves are
    // multiples of 4).
    const long nitems = base < total ? (total - base + nwaves - 1) / nwaves : 0;
    int* table = reinterpret_cast<int*>(ring + RG::kBytes);

    for (long k0 = 0; k0 < nitems; k0 += kTable) {
        const int cnt = (int)min((long)kTable, nitems - k0);
        fill_table(a, table, base, nwaves, nfb, k0, cnt);
        __syncthreads();
        const long nsteps = (long)cnt * nbatch;

        // Prologue: batches 0 .. D-2 in flight.
        int iss_k = 0, iss_b = 0;
        Item iss = item_from_table<NMAT>(a, table, 0, wave, nfb, KG);
        for (int j = 0; j < D - 1; ++j) {
            if (j < nsteps) {
                issue_batch<NMAT, PF, D>(a, iss, iss_b, K, KG, ring + (j % D) * RG::kSlot, wave,
                                         lane);
                if (++iss_b == nbatch) {
                    iss_b = 0;
                    if (++iss_k < cnt) iss = item_from_table<NMAT>(a, table, iss_k, wave, nfb, KG);
                }
            }
        }

        int cur_k = 0, cur_b = 0;
        Item cur = item_from_table<NMAT>(a, table, 0, wave, nfb, KG);
        f32x4 acc[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};

        for (long step = 0; step < nsteps; ++step) {
            // Batch `step` has landed once at most (D-2) newer batches are pending.
            if (step + D - 2 < nsteps) wait_vmcnt<RG::kDma * (D - 2)>();
            else wait_vmcnt<0>();
            __builtin_amdgcn_s_barrier();
            if (step + D - 1 < nsteps) {
                issue_batch<NMAT, PF, D>(a, iss, iss_b, K, KG,
                                         ring + ((step + D - 1) % D) * RG::kSlot, wave, lane);
                if (++iss_b == nbatch) {
                    iss_b = 0;
                    if (++iss_k < cnt) iss = item_from_table<NMAT>(a, table, iss_k, wave, nfb, KG);
                }
            }
            compute_batch<NMAT, PF, D>(ring + (step % D) * RG::kSlot, cur_b, KG, wave, lane, dqc,
                                       acc);

            if (++cur_b == nbatch) {
                const bool valid = r < cur.nr;
                const size_t row = (size_t)cur.r0 + r;
                if constexpr (NMAT == 2) {
                    uint32_t hb[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        hb[j] = f32_to_bf16(silu_fast(acc[0][j]) * acc[1][j]);
                    if (valid) {
                        uint2 v = {hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16)};
                        *reinterpret_cast<uint2*>(a.h + row * a.I + cur.fb * 16 + 4 * q) = v;
                    }
                } else {
                    if (valid)
                        *reinterpret_cast<float4*>(a.dpart + row * a.H + cur.fb * 16 + 4 * q) =
                            make_float4(acc[0][0], acc[0][1], acc[0][2], acc[0][3]);
                }
#pragma unroll
                for (int m = 0; m < NMAT; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
                cur_b = 0;
                if (++cur_k < cnt) cur = item_from_table<NMAT>(a, table, cur_k, wave, nfb, KG);
            }
        }
        // All DMA has landed (the last step waited vmcnt(0)); every wave is
        // done reading the ring and the table before the next chunk refills.
        __syncthreads();
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
// Ring depth per projection; both fit the 160 KiB of LDS of one workgroup.
// Batches of 2 groups keep two 4-wave workgroups resident per CU (8 waves).
constexpr int kRingGU = 3;
constexpr int kRingDown = 4;
constexpr int kPFGU = 2;
constexpr int kPFDown = 2;

template <int NMAT, int PF, int D>
static int launch_expert(const ExpArgs& a, long max_work, hipStream_t s) {
    using RG = Ring<NMAT, PF, D>;
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&w4_expert_kernel<NMAT, PF, D>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, RG::kTotal) !=
            hipSuccess)
            return -4;
        attr_set = true;
    }
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    // As many workgroups as fit in LDS at once; persistent over items.
    const int per_cu = (160 * 1024) / RG::kTotal;
    long blocks = (max_work + 3) / 4;
    if (blocks > (long)cus * per_cu) blocks = (long)cus * per_cu;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL((w4_expert_kernel<NMAT, PF, D>), dim3((unsigned)blocks), dim3(256),
                       RG::kTotal, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_gate_up(const ExpertPtrs& P, const uint16_t* x, const int* tiles, const int* ntiles,
                   int max_tiles, const int* rows_tok, uint16_t* h, int H, int I, int E,
                   hipStream_t s) {
    ExpArgs a{};
    a.wq[0] = reinterpret_cast<const uint4*>(P.gate_q); a.ws[0] = P.gate_s;
    a.wq[1] = reinterpret_cast<const uint4*>(P.up_q); a.ws[1] = P.up_s;
    a.swq[0] = reinterpret_cast<const uint4*>(P.sh_gate_q); a.sws[0] = P.sh_gate_s;
    a.swq[1] = reinterpret_cast<const uint4*>(P.sh_up_q); a.sws[1] = P.sh_up_s;
    a.src = x; a.tiles = reinterpret_cast<const int4*>(tiles); a.ntiles = ntiles;
    a.rows_tok = rows_tok; a.h = h; a.H = H; a.I = I; a.E = E;
    return launch_expert<2, kPFGU, kRingGU>(a, (long)max_tiles * (I / 16), s);
}

int launch_down(const ExpertPtrs& P, const uint16_t* h, const int* tiles, const int* ntiles,
                int max_tiles, float* dpart, int H, int I, int E, hipStream_t s) {
    ExpArgs a{};
    a.wq[0] = reinterpret_cast<const uint4*>(P.down_q); a.ws[0] = P.down_s;
    a.swq[0] = reinterpret_cast<const uint4*>(P.sh_down_q); a.sws[0] = P.sh_down_s;
    a.wq[1] = a.wq[0]; a.ws[1] = a.ws[0]; a.swq[1] = a.swq[0]; a.sws[1] = a.sws[0];
    a.src = h; a.tiles = reinterpret_cast<const int4*>(tiles); a.ntiles = ntiles;
    a.dpart = dpart; a.H = H; a.I = I; a.E = E;
    return launch_expert<1, kPFDown, kRingDown>(a, (long)max_tiles * (H / 16), s);
}

int launch_combine(const float* dpart, const int* inv, const float* w, int n, int topk, int H,
                   int with_shared, float* out, hipStream_t s) {
    dim3 grid((unsigned)((H / 4 + 255) / 256), (unsigned)n);
    hipLaunchKernelGGL(combine_kernel, grid, dim3(256), 0, s, dpart, inv, w, n, topk, H,
                       with_shared, out);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace glmmoe
