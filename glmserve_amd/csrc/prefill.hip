// W4A16 experts, large-group regime (prefill and wide verify batches):
// grouped GEMM tiles of up to 128 grouped rows x 256 weight rows on bf16
// MFMA 32x32x16.
//
// Reference: the expert-major tensor-core path of the reference's GGUF MoE
// (cuda/qgemm.cu:1269-1356, emajor_mma_s8_kernel, used once n*topk reaches
// GLMSERVE_MMA_MOE_MIN_TS) and its W4A16 expert FFN semantics
// (cuda/moe_expert.cu:143-222).
//
// Work item = (row tile, feature group). A workgroup of 8 waves computes
// 128 rows x 256 weight rows: for gate/up 128 features (the gate rows and the
// up rows of the same features, one 128-feature group of h), for down 256
// features. Wave w owns ALL 128 rows (4 row blocks of 32, the MFMA A operand)
// and 32 weight rows (the B operand): for gate/up 16 gate + the same 16 up
// features, for down 32 features. So every weight element is decoded once
// per workgroup, and a lane's output column is one weight row with one scale
// per 128-K group.
//
// Streams, per 128-K group g:
// - activations: the 128 rows (gathered by token for gate/up) x 256 B go
//   global -> LDS by LDS-DMA (buffer loads: the per-group step is a scalar
//   offset, so issuing costs no VALU) into a 4-slot ring, issued three groups
//   ahead. A row occupies 272 B of its slot (16 B of padding), so the 16 rows
//   of a fragment read fall on 16 distinct bank groups and every fragment
//   address is the lane's base plus an immediate offset;
// - weights: each lane loads its own 32 B of int4 (two dwordx4) straight into
//   registers, four groups ahead (a 4-deep register ring);
// - per batch of 8 groups: the scales of the workgroup's 16 weight tiles and
//   the 8 group sums of each row, one DMA per wave into double buffers.
// One s_barrier per group, in the middle of the group, publishes slot g + 1
// (every wave waited for its own DMAs of g + 1) and frees slot g - 1 for
// group g + 3.
//
// Arithmetic. The int4 code c decodes exactly to the bf16 of 128 + c
// (dq_w4), so a group's MFMAs give P = sum_k (128 + c) x = sum_k (c - 8) x
// + 136 X with X the row's group sum. acc += s * P per group (one fma per
// element, s the column's bf16 scale), and once per 8 groups one MFMA adds
// sum_g s_g * (-136 X_g) for all 8 groups: its A operand holds -136 X_g split
// into bf16 hi + lo parts (exact to 2^-16 relative), its B operand s_g twice.
//
// Schedule of a group's 32 MFMAs (4 row blocks x 8 K-steps): quarters
// Q1 = blocks 0,1 steps 0-3, Q2 = blocks 2,3 steps 0-3, Q3 = blocks 0,1
// steps 4-7, Q4 = blocks 2,3 steps 4-7. The VALU work spreads evenly: Q1
// rescales blocks 2,3 of the previous group, Q2 decodes steps 4-7 of this
// group's weights, Q3 decodes steps 0-3 of the next group's, Q4 rescales
// blocks 0,1. LDS fragments are read one step ahead. Row blocks past the
// tile's last row skip their MFMAs and fragment reads (an expert's last tile
// is often short), and keep the VALU work.
#include "common.hpp"
#include "bigtile.hpp"
#include "kernels.hpp"

namespace glmmoe {

struct MmArgs {
    const uint8_t* wq[2];     // packed int4 tiles of the routed experts (gate, up) or (down, -)
    const uint16_t* ws[2];    // bf16 scales [rows/16][K/128][16]
    const uint8_t* swq[2];    // the shared expert's
    const uint16_t* sws[2];
    const uint16_t* src;      // x [n, H] (gate/up, rows gathered by token) or h [R, I] (down)
    const float* gsum;        // xsum [n, H/128] or hsum [R, I/128]
    const int4* tiles; const int* ntiles; const int* rows_tok;
    uint16_t* h; float* hsum;   // gate/up outputs
    uint16_t* dout;             // down output: bf16 [R, H]
    int H, I, E;
};

namespace mm {
constexpr int kRowB = 272;                     // LDS bytes per activation row (256 + 16 padding)
constexpr int kSlot = 128 * kRowB;             // 34 KiB: 34 DMAs of 1 KiB
constexpr int kDmas = kSlot / 1024;
constexpr int kRing = 4;
constexpr int kXBuf = kRing * kSlot;           // 2 x 4 KiB: [row][8 groups] fp32
constexpr int kSBuf = kXBuf + 2 * 4096;        // 2 x 4 KiB: [tile 16][group 8][row 16] bf16
constexpr int kTab = kSBuf + 2 * 4096;
constexpr int kTabItems = 8;
constexpr int kTotal = kTab + kTabItems * kBigTabInts * 4;
static_assert(kTotal <= 160 * 1024, "one workgroup's LDS");
constexpr int kBlk = 32 * kRowB;               // one 32-row block
}  // namespace mm

// Weight tile of lane column col for wave w, feature group g.
//   gate/up: matrix col >> 4 (0 gate, 1 up), 16-row block 8 g + w;
//   down:    matrix 0, block 16 g + 2 w + (col >> 4).
template <int NMAT>
__device__ __forceinline__ void mm_lane_tile(int g, int wave, int col, int& m, int& fb) {
    if (NMAT == 2) {
        m = col >> 4;
        fb = 8 * g + wave;
    } else {
        m = 0;
        fb = 16 * g + 2 * wave + (col >> 4);
    }
}
// Index of lane column col's tile in the scale buffer (gate tiles 0-7, up 8-15).
template <int NMAT>
__device__ __forceinline__ int mm_sbuf_tile(int wave, int col) {
    return NMAT == 2 ? 8 * (col >> 4) + wave : 2 * wave + (col >> 4);
}

template <int NMAT>
__device__ __forceinline__ const uint8_t* mm_wbase(const MmArgs& a, int e, int m, int frows, int KG) {
    const size_t stride = (size_t)(frows / 16) * KG * 1024;
    return e == a.E ? a.swq[m] : a.wq[m] + (size_t)e * stride;
}
template <int NMAT>
__device__ __forceinline__ const uint16_t* mm_sbase(const MmArgs& a, int e, int m, int frows, int KG) {
    const size_t stride = (size_t)(frows / 16) * KG * 16;
    return e == a.E ? a.sws[m] : a.ws[m] + (size_t)e * stride;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t mm_rsrc(const void* base) {
    // Raw buffer over 4 GiB - 1 from base (no stride, no swizzle).
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)0xffffffffu,
                                             0x00020000);
}

// Per-lane stream state of one item.
//   act[i]: byte offset (in src) of this lane's 16 B of activation DMA i at
//     group 0; DMA d = wave + 8 i (and d = 32 + wave for waves 0, 1) fills
//     slot bytes 1024 d + 16 lane = row p / 17, 16-B chunk p % 17 (p = 64 d +
//     lane); chunk 16 is padding (loads chunk 0 again);
//   w: the lane's 32 B of int4 at group 0 (K positions 64 h .. 64 h + 63 of
//     weight row col % 16 of its tile);
//   bt: byte offset of the lane's 16 B of the batch DMA at batch 0 (waves 0-3:
//     group sums of row 32 w + lane / 2, groups 4 (lane & 1) + [0, 4); waves
//     4-7: 16 B of scales of tile 4 (w - 4) + lane / 16).
struct MmPtrs {
    uint32_t act[5];
    const uint4* w;
    uint32_t bt;
};
struct MmUni {            // the same, wave-uniform parts
    const uint16_t* sbt;  // waves 4-7: the scale matrix the batch DMA reads
    int nrb;              // live 32-row blocks of the item
};

template <int NMAT>
__device__ __forceinline__ MmPtrs mm_ptrs(const MmArgs& a, const BigItem& it, int K, int KG, int wave,
                                          int lane, MmUni& u) {
    MmPtrs p;
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        const int d = i < 4 ? wave + 8 * i : 32 + (wave & 1);
        const int pos = 64 * d + lane;
        const int row = pos / 17, c = pos % 17;
        p.act[i] = lds_read32(it.tab + 16 + row * 4) * (uint32_t)(K * 2) + (uint32_t)((c & 15) * 16);
    }
    const int col = lane & 31, h = lane >> 5;
    const int frows = NMAT == 2 ? a.I : a.H;
    {
        int m, fb;
        mm_lane_tile<NMAT>(it.g, wave, col, m, fb);
        const uint4* base = reinterpret_cast<const uint4*>(mm_wbase<NMAT>(a, it.e, m, frows, KG));
        p.w = base + (size_t)fb * KG * 64 + (col & 15) + 32 * h;
    }
    if (wave < 4) {
        const int row = wave * 32 + (lane >> 1);
        p.bt = (lds_read32(it.tab + 16 + row * 4) * (uint32_t)KG + 4u * (lane & 1)) * 4u;
        u.sbt = nullptr;
    } else {
        const int t = 4 * (wave - 4) + (lane >> 4);
        const int m = NMAT == 2 ? (t >> 3) : 0;
        const int fb = NMAT == 2 ? 8 * it.g + (t & 7) : 16 * it.g + t;
        u.sbt = mm_sbase<NMAT>(a, it.e, m, frows, KG);
        p.bt = ((uint32_t)fb * KG * 16 + (lane & 15) * 8) * 2u;
    }
    u.nrb = (it.nr + 31) >> 5;
    return p;
}

// bf16 pair {hi(v), bf16(v - hi(v))} as one dword (hi in the low half).
__device__ __forceinline__ uint32_t split_bf16(float v) {
    const float hi = __uint_as_float(__float_as_uint(v) & 0xffff0000u);
    return pack_bf16x2(hi, v - hi);
}

// Fragments of two row blocks: OFF and OFF + one block past addr.
template <int OFF>
__device__ __forceinline__ void lds_read2(uint32_t addr, u32x4& a, u32x4& b) {
    asm volatile("ds_read_b128 %0, %2 offset:%3\n ds_read_b128 %1, %2 offset:%4"
                 : "=&v"(a), "=&v"(b)
                 : "v"(addr), "n"(OFF), "n"(OFF + mm::kBlk));
}
template <int N>
__device__ __forceinline__ void lgkm_wait(u32x4& a, u32x4& b) {
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N));
}

__device__ __forceinline__ void dma_buf16(__amdgpu_buffer_rsrc_t r, uint32_t lds_dst, uint32_t voff,
                                          uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)(uintptr_t)lds_dst, 16, voff, soff, 0, 0);
}

// Stores an item's outputs. red: 4 KiB of LDS free for the call (the hsum
// partials of gate/up).
template <int NMAT>
__device__ __forceinline__ void mm_epilogue(const MmArgs& a, const BigItem& cur, uint32_t red, int wave,
                                            int lane, f32x16 (&acc)[4]) {
    // Laundered lane index: keeps the per-row addresses below from being
    // hoisted out of the streaming loop (they would stay live and spill).
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int col = ln & 31, h = ln >> 5;
    if constexpr (NMAT == 2) {
        // Lanes col < 16 hold gate features, col >= 16 the same up features.
        // Each lane of a pair forms h for half of the values: col < 16 the
        // values i < 8 of every row block, col >= 16 the values i >= 8.
        const bool lo = col < 16;
        const int f = cur.g * 128 + wave * 16 + (col & 15);
        uint16_t* hcol = a.h + (size_t)cur.r0 * a.I + f;
        float v[32];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float send = lo ? acc[rb][i + 8] : acc[rb][i];
                const float recv = __shfl_xor(send, 16);
                const float gt = lo ? acc[rb][i] : recv;
                const float up = lo ? recv : acc[rb][i + 8];
                const uint32_t hb = pack_bf16x2(silu_fast(gt) * up, 0.0f) & 0xffffu;
                const int ii = lo ? i : i + 8;
                const int row = rb * 32 + 8 * (ii >> 2) + 4 * h + (ii & 3);
                if (row < cur.nr) hcol[(size_t)row * a.I] = (uint16_t)hb;
                v[rb * 8 + i] = bf16_to_f32(hb);
            }
        // Row sums over the 16 features of the lane's 16-lane row group
        // (fixed recursive halving: lane c ends with the sums of values
        // 2 (c % 16) and 2 (c % 16) + 1), then over the 8 waves in order.
        const int c = col & 15;
        auto halve = [&](auto N_) {
            constexpr int N = decltype(N_)::value;
            const bool upper = (c & N) != 0;
#pragma unroll
            for (int j = 0; j < 2 * N; ++j) {
                const float send = upper ? v[j] : v[j + 2 * N];
                const float keep = upper ? v[j + 2 * N] : v[j];
                v[j] = keep + __shfl_xor(send, N);
            }
        };
        halve(std::integral_constant<int, 8>{});
        halve(std::integral_constant<int, 4>{});
        halve(std::integral_constant<int, 2>{});
        halve(std::integral_constant<int, 1>{});
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int idx = 2 * c + q;                       // value index rb * 8 + i
            const int rb = idx >> 3, i = idx & 7;
            const int ii = lo ? i : i + 8;
            const int row = rb * 32 + 8 * (ii >> 2) + 4 * h + (ii & 3);
            lds_write32(red + (uint32_t)((wave * 128 + row) * 4), v[q]);
        }
        __builtin_amdgcn_s_barrier();
        if (wave == 0) {
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int row = half * 64 + ln;
                float s = 0.0f;
#pragma unroll
                for (int w = 0; w < 8; ++w) s += __uint_as_float(lds_read32(red + (uint32_t)((w * 128 + row) * 4)));
                if (row < cur.nr) a.hsum[((size_t)cur.r0 + row) * (a.I / 128) + cur.g] = s;
            }
        }
        __builtin_amdgcn_s_barrier();   // partials read before the next item reuses them
    } else {
        // Per-row expert outputs as bf16 (the combine adds them in fp32).
        uint16_t* dcol = a.dout + (size_t)cur.r0 * a.H + cur.g * 256 + wave * 32 + col;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = rb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
                if (row < cur.nr) dcol[(size_t)row * a.H] = (uint16_t)(pack_bf16x2(acc[rb][i], 0.0f) & 0xffffu);
            }
    }
}

template <int NMAT>
__global__ __launch_bounds__(512) void w4_mm_kernel(MmArgs a) {
    extern __shared__ __align__(16) char lds[];
    const DqConst dqc = dq_const();
    int* table = reinterpret_cast<int*>(lds + mm::kTab);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 31, h = lane >> 5;
    const int K = NMAT == 2 ? a.H : a.I;
    const int KG = K / 128;          // a multiple of 8 (checked by the launcher)
    const int NB = KG / 8;           // batches per item
    const int nfg = NMAT == 2 ? a.I / 128 : a.H / 256;
    // Tile classes (dispatch order): full tiles [0, nt4), then each expert's
    // last tile of 33-64 rows [nt4, nt2), then of at most 32 rows [nt2, nt):
    // 4, 2 and 1 live 32-row blocks.
    const int nt = a.ntiles[0], nt4 = a.ntiles[1], nt2 = a.ntiles[2];
    const long nitems = big_rounds((long)nt * nfg);
    const uint32_t ring = lds_addr(lds);
    // Lane's fragment address at step 0 of row block 0 in slot 0: row col,
    // 16-B chunk 8 h; step s adds 16 s, row block rb 8704 rb, slot q 34 KiB q.
    const uint32_t xa0 = ring + (uint32_t)(col * mm::kRowB + h * 128);
    const int stile = mm_sbuf_tile<NMAT>(wave, col);
    const __amdgpu_buffer_rsrc_t rsrc_src = mm_rsrc(a.src);
    const __amdgpu_buffer_rsrc_t rsrc_x = mm_rsrc(a.gsum);

    // A workgroup's items come in increasing id order, so class by class.
    // Each chunk of at most kTabItems items of one class runs one pipeline
    // (prologue, stream, drain) specialized to its live row blocks: the
    // accumulators never cross from one specialization to another.
    auto cls_of = [&](long k) {
        const long t = big_item_id(k) / nfg;
        return t < nt4 ? 4 : t < nt2 ? 2 : 1;
    };
    auto run_chunk = [&](auto NRB_, long k0, int cnt) {
        constexpr int NRB = decltype(NRB_)::value;
        constexpr bool live1 = NRB > 1, live23 = NRB > 2, live3 = NRB > 3;
        big_fill_table<NMAT == 2>(a.tiles, a.rows_tok, table, k0, cnt, nfg);
        __syncthreads();
        const int NBt = cnt * NB;        // batches of this chunk
        auto item = [&](int k) { return big_item(lds + mm::kTab, k < cnt ? k : cnt - 1); };

        // Stream state of the item of the current batch (pc) and of the next
        // item (pn; past the chunk's end the last item again: those loads
        // land in buffers nobody reads). In the last batch of an item the
        // activation stream (3 groups ahead) and the weight stream (4 ahead)
        // cross into the next item at fixed group positions.
        MmUni uc, un;
        MmPtrs pc = mm_ptrs<NMAT>(a, item(0), K, KG, wave, lane, uc);
        MmPtrs pn = mm_ptrs<NMAT>(a, item(1), K, KG, wave, lane, un);
        // Five activation DMAs per wave per group, so every wave waits for
        // the same counts: DMAs 32 and 33 (waves 0, 1) are repeated by waves
        // 2-7 (same source, same LDS bytes). No branch may sit in the
        // unrolled group body: the compiler then spills the accumulators.
        auto issue_act = [&](const MmPtrs& p, int k, int gslot) {
            const uint32_t dst = ring + (uint32_t)((gslot & 3) * mm::kSlot);
            const uint32_t soff = (uint32_t)k * 256u;
#pragma unroll
            for (int i = 0; i < 4; ++i) dma_buf16(rsrc_src, dst + (uint32_t)((wave + 8 * i) * 1024), p.act[i], soff);
            dma_buf16(rsrc_src, dst + (uint32_t)((32 + (wave & 1)) * 1024), p.act[4], soff);
        };
        u32x4 W[4][2];
        auto issue_w = [&](const uint4* pw, int k, int r) {
            const uint4* q = pw + (size_t)k * 64;
            W[r][0] = __builtin_bit_cast(u32x4, q[0]);
            W[r][1] = __builtin_bit_cast(u32x4, q[16]);
        };
        auto issue_batch = [&](uint32_t bt, const uint16_t* sbt, int kb, int parity) {
            // Waves 0-3: group sums; waves 4-7: scales (selects, no branch).
            const bool xw = wave < 4;
            const __amdgpu_buffer_rsrc_t r = xw ? rsrc_x : mm_rsrc(sbt);
            const uint32_t dst = xw ? lds_addr(lds + mm::kXBuf + parity * 4096 + wave * 1024)
                                    : lds_addr(lds + mm::kSBuf + parity * 4096 + (wave - 4) * 1024);
            dma_buf16(r, dst, bt, (uint32_t)kb * (xw ? 32u : 256u));
        };

        // Prologue: batch 0, activation groups 0-2, weight groups 0-3.
        issue_batch(pc.bt, uc.sbt, 0, 0);
        issue_act(pc, 0, 0);
        issue_act(pc, 1, 1);
        issue_act(pc, 2, 2);
#pragma unroll
        for (int r = 0; r < 4; ++r) issue_w(pc.w, r, r);
        wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();

        f32x16 acc[4], P[4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) acc[rb] = f32x16{};
        bf16x8 Bd[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) Bd[s] = dq_w4(W[0][s >> 2][s & 3], dqc);
        // Fragments of Q1 step 0 (row blocks 0, 1 of slot 0).
        u32x4 A[2][2];
        lds_read2<0>(xa0, A[0][0], A[0][1]);
        float sc_prev = 0.0f;
        int ib = 0, kb = 0;   // item and batch-in-item of the current batch

        for (int b = 0; b < NBt; ++b) {
            const bool last = kb == NB - 1;
            // Liveness is a compile-time constant of the chunk: an MFMA under
            // a run-time branch makes the compiler copy whole accumulators.
            static_for<8>([&](auto J) {
                constexpr int j = decltype(J)::value;
                // Fragment base of slot g and g + 1 (an opaque scalar offset,
                // so the per-slot bases are formed here, not precomputed).
                uint32_t so = (uint32_t)((j & 3) * mm::kSlot), nso = (uint32_t)(((j + 1) & 3) * mm::kSlot);
                asm volatile("" : "+s"(so), "+s"(nso));
                const uint32_t xg = xa0 + so;
                // ---- Q1: row blocks 0, 1, steps 0-3; rescale blocks 2, 3 of g - 1.
                static_for<4>([&](auto S_) {
                    constexpr int s = 0 + decltype(S_)::value;
                    constexpr int cb = s & 1, nb = cb ^ 1;
                    if constexpr (s < 3) lds_read2<16 * (s + 1)>(xg, A[nb][0], A[nb][1]);
                    else if constexpr (live23) lds_read2<2 * mm::kBlk>(xg, A[nb][0], A[nb][1]);
                    else lds_read2<16 * 4>(xg, A[nb][0], A[nb][1]);
                    lgkm_wait<2>(A[cb][0], A[cb][1]);
                    P[0] = mfma32x32x16(as_bf16x8(A[cb][0]), Bd[s], s == 0 ? f32x16{} : P[0]);
                    if constexpr (live1) P[1] = mfma32x32x16(as_bf16x8(A[cb][1]), Bd[s], s == 0 ? f32x16{} : P[1]);
                    if constexpr (j > 0) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const int blk = 2 + (e >> 2), idx = s * 4 + (e & 3);
                            acc[blk][idx] = __builtin_fmaf(sc_prev, P[blk][idx], acc[blk][idx]);
                        }
                    }
                });
                // ---- Q2: row blocks 2, 3, steps 0-3; decode steps 4-7 of g's weights.
                if constexpr (live23) {
                static_for<4>([&](auto S_) {
                        constexpr int s = 0 + decltype(S_)::value;
                        constexpr int cb = (s + 4) & 1, nb = cb ^ 1;
                        if constexpr (s < 3) lds_read2<2 * mm::kBlk + 16 * (s + 1)>(xg, A[nb][0], A[nb][1]);
                        else lds_read2<16 * 4>(xg, A[nb][0], A[nb][1]);
                        lgkm_wait<2>(A[cb][0], A[cb][1]);
                        P[2] = mfma32x32x16(as_bf16x8(A[cb][0]), Bd[s], s == 0 ? f32x16{} : P[2]);
                        if constexpr (live3) P[3] = mfma32x32x16(as_bf16x8(A[cb][1]), Bd[s], s == 0 ? f32x16{} : P[3]);
                        Bd[4 + s] = dq_w4(W[j & 3][1][s], dqc);
                    });
                } else {
#pragma unroll
                    for (int s = 0; s < 4; ++s) Bd[4 + s] = dq_w4(W[j & 3][1][s], dqc);
                }
                // ---- mid-group: publish slot g + 1, free slot g - 1, issue.
                // Pending before the wait: this wave's DMAs of g + 1 (issued at
                // g - 2) and everything after them: the weights of g + 2 (+ the
                // batch DMA if g - 2 opened a batch) and the whole issue of g - 1
                // (5 activation DMAs, 2 weight loads, maybe the batch DMA).
                {
                    constexpr int n2 = 2 + (((j + 6) & 7) == 0 ? 1 : 0);
                    constexpr int n1 = 7 + (((j + 7) & 7) == 0 ? 1 : 0);
                    wait_vmcnt<n2 + n1>();
                }
                __builtin_amdgcn_s_barrier();
                // Stream sources: activations of group g + 3, weights of group
                // g + 4 (this item's or, late in its last batch, the next
                // item's: selects, no branches). The 5 activation DMAs, the
                // weight loads and the batch DMA are spread over Q3 and Q4, one
                // per step, so their issue overlaps the MFMAs instead of
                // stalling all waves together after the barrier.
                MmPtrs pa = pc;
                int ka = 8 * kb + j + 3;
                if constexpr (j >= 5) {
#pragma unroll
                    for (int q = 0; q < 5; ++q) pa.act[q] = last ? pn.act[q] : pc.act[q];
                    ka = last ? j - 5 : ka;
                }
                const uint4* pw = pc.w;
                int kw = 8 * kb + j + 4;
                if constexpr (j >= 4) {
                    pw = last ? pn.w : pc.w;
                    kw = last ? j - 4 : kw;
                }
                const uint32_t adst = ring + (uint32_t)(((j + 3) & 3) * mm::kSlot);
                const uint32_t asoff = (uint32_t)ka * 256u;
                auto issue_part = [&](auto IP_) {
                    constexpr int ip = decltype(IP_)::value;
                    if constexpr (ip < 4) {
                        dma_buf16(rsrc_src, adst + (uint32_t)((wave + 8 * ip) * 1024), pa.act[ip], asoff);
                    } else if constexpr (ip == 4) {
                        dma_buf16(rsrc_src, adst + (uint32_t)((32 + (wave & 1)) * 1024), pa.act[4], asoff);
                    } else if constexpr (ip == 5) {
                        issue_w(pw, kw, (j + 4) & 3);
                    } else if constexpr (ip == 6 && j == 0) {
                        issue_batch(last ? pn.bt : pc.bt, last ? un.sbt : uc.sbt, last ? 0 : kb + 1, (b + 1) & 1);
                    }
                };
                // The scale of this lane's column for group g (waited for with
                // Q3's first fragments).
                uint32_t scr;
                asm volatile("ds_read_u16 %0, %1"
                             : "=v"(scr)
                             : "v"(lds_addr(lds + mm::kSBuf + (b & 1) * 4096 + stile * 256 + j * 32) +
                                   (uint32_t)((col & 15) * 2)));
                // ---- Q3: row blocks 0, 1, steps 4-7; decode steps 0-3 of g + 1.
                static_for<4>([&](auto S_) {
                    constexpr int s = 4 + decltype(S_)::value;
                    constexpr int cb = s & 1, nb = cb ^ 1;
                    if constexpr (s < 7) lds_read2<16 * (s + 1)>(xg, A[nb][0], A[nb][1]);
                    else if constexpr (live23) lds_read2<2 * mm::kBlk + 16 * 4>(xg, A[nb][0], A[nb][1]);
                    else lds_read2<0>(xa0 + nso, A[nb][0], A[nb][1]);
                    if constexpr (s == 4) asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(A[cb][0]), "+v"(A[cb][1]), "+v"(scr));
                    else lgkm_wait<2>(A[cb][0], A[cb][1]);
                    P[0] = mfma32x32x16(as_bf16x8(A[cb][0]), Bd[s], P[0]);
                    if constexpr (live1) P[1] = mfma32x32x16(as_bf16x8(A[cb][1]), Bd[s], P[1]);
                    Bd[s - 4] = dq_w4(W[(j + 1) & 3][0][s - 4], dqc);
                    issue_part(std::integral_constant<int, s - 4>{});
                });
                const float sc = bf16_to_f32(scr);
                // ---- Q4: row blocks 2, 3, steps 4-7; rescale blocks 0, 1 of g.
                if constexpr (live23) {
                static_for<4>([&](auto S_) {
                        constexpr int s = 4 + decltype(S_)::value;
                        constexpr int cb = (s + 4) & 1, nb = cb ^ 1;
                        // next: Q4 step s + 1, or Q1 step 0 of g + 1 (next slot)
                        if constexpr (s < 7) lds_read2<2 * mm::kBlk + 16 * (s + 1)>(xg, A[nb][0], A[nb][1]);
                        else lds_read2<0>(xa0 + nso, A[nb][0], A[nb][1]);
                        lgkm_wait<2>(A[cb][0], A[cb][1]);
                        P[2] = mfma32x32x16(as_bf16x8(A[cb][0]), Bd[s], P[2]);
                        if constexpr (live3) P[3] = mfma32x32x16(as_bf16x8(A[cb][1]), Bd[s], P[3]);
                        issue_part(std::integral_constant<int, s>{});
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const int blk = e >> 2, idx = (s - 4) * 4 + (e & 3);
                            acc[blk][idx] = __builtin_fmaf(sc, P[blk][idx], acc[blk][idx]);
                        }
                    });
                } else {
                    issue_part(std::integral_constant<int, 4>{});
                    issue_part(std::integral_constant<int, 5>{});
                    issue_part(std::integral_constant<int, 6>{});
#pragma unroll
                    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
                        for (int i = 0; i < 16; ++i) acc[blk][i] = __builtin_fmaf(sc, P[blk][i], acc[blk][i]);
                }
                sc_prev = sc;
            });

            // ---- end of batch: rescale blocks 2, 3 of the last group, then
            // the batch's offset correction.
#pragma unroll
            for (int blk = 2; blk < 4; ++blk)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[blk][i] = __builtin_fmaf(sc_prev, P[blk][i], acc[blk][i]);
            {
                const uint32_t xb = lds_addr(lds + mm::kXBuf + (b & 1) * 4096);
                const uint32_t sb = lds_addr(lds + mm::kSBuf + (b & 1) * 4096 + stile * 256) +
                                    (uint32_t)((col & 15) * 2);
                uint32_t sv[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) sv[q] = lds_read_u16(sb + (uint32_t)((4 * h + q) * 32));
                const bf16x8 sop = __builtin_bit_cast(
                    bf16x8, u32x4{sv[0] | (sv[0] << 16), sv[1] | (sv[1] << 16), sv[2] | (sv[2] << 16),
                                  sv[3] | (sv[3] << 16)});
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) {
                    const uint4 xv = lds_bcast16(xb + (uint32_t)((rb * 32 + col) * 32 + h * 16));
                    const bf16x8 xop = __builtin_bit_cast(
                        bf16x8, u32x4{split_bf16(-136.0f * __uint_as_float(xv.x)),
                                      split_bf16(-136.0f * __uint_as_float(xv.y)),
                                      split_bf16(-136.0f * __uint_as_float(xv.z)),
                                      split_bf16(-136.0f * __uint_as_float(xv.w))});
                    acc[rb] = mfma32x32x16(xop, sop, acc[rb]);
                }
            }
            if (last) {
                // Item done: store it (the fragments of the next group's Q1
                // step 0 are in flight in A[0]; wait for them first). The
                // epilogue's LDS scratch is this batch's scale buffer, consumed
                // above and next written by the batch DMA of the next batch.
                lgkm_wait<0>(A[0][0], A[0][1]);
                __builtin_amdgcn_s_barrier();   // every wave has read this batch's scales
                mm_epilogue<NMAT>(a, item(ib), lds_addr(lds + mm::kSBuf + (b & 1) * 4096), wave, lane, acc);
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) acc[rb] = f32x16{};
                ++ib;
                kb = 0;
                pc = pn;
                uc = un;
                pn = mm_ptrs<NMAT>(a, item(ib + 1), K, KG, wave, lane, un);
            } else {
                ++kb;
            }
        }
        wait_vmcnt<0>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
    };
    for (long k0 = 0; k0 < nitems;) {
        const int cls = cls_of(k0);
        int cnt = 1;
        while (cnt < mm::kTabItems && k0 + cnt < nitems && cls_of(k0 + cnt) == cls) ++cnt;
        if (cls == 4) run_chunk(std::integral_constant<int, 4>{}, k0, cnt);
        else if (cls == 2) run_chunk(std::integral_constant<int, 2>{}, k0, cnt);
        else run_chunk(std::integral_constant<int, 1>{}, k0, cnt);
        k0 += cnt;
    }
}

template <int NMAT>
static int launch_mm(const MmArgs& a, long max_items, hipStream_t s) {
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&w4_mm_kernel<NMAT>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, mm::kTotal) != hipSuccess)
            return -4;
        attr_set = true;
    }
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    long blocks = max_items < cus ? max_items : cus;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL((w4_mm_kernel<NMAT>), dim3((unsigned)blocks), dim3(512), mm::kTotal, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

bool big_w4_shape_ok(int H, int I) { return H % 1024 == 0 && I % 1024 == 0; }

int launch_gate_up_big(const ExpertPtrs& P, const uint16_t* x, const float* xsum,
                       const int* tiles, const int* ntiles, int max_tiles, const int* rows_tok,
                       uint16_t* h, float* hsum, int H, int I, int E, hipStream_t s) {
    if (!big_w4_shape_ok(H, I)) return -2;
    MmArgs a{};
    a.wq[0] = P.gate_q; a.ws[0] = P.gate_s; a.wq[1] = P.up_q; a.ws[1] = P.up_s;
    a.swq[0] = P.sh_gate_q; a.sws[0] = P.sh_gate_s; a.swq[1] = P.sh_up_q; a.sws[1] = P.sh_up_s;
    a.src = x; a.gsum = xsum; a.tiles = reinterpret_cast<const int4*>(tiles); a.ntiles = ntiles;
    a.rows_tok = rows_tok; a.h = h; a.hsum = hsum; a.H = H; a.I = I; a.E = E;
    return launch_mm<2>(a, (long)max_tiles * (I / 128), s);
}

int launch_down_big(const ExpertPtrs& P, const uint16_t* h, const float* hsum, const int* tiles,
                    const int* ntiles, int max_tiles, float* dpart, int H, int I, int E,
                    hipStream_t s) {
    if (!big_w4_shape_ok(H, I)) return -2;
    MmArgs a{};
    a.wq[0] = P.down_q; a.ws[0] = P.down_s; a.wq[1] = P.down_q; a.ws[1] = P.down_s;
    a.swq[0] = P.sh_down_q; a.sws[0] = P.sh_down_s; a.swq[1] = P.sh_down_q; a.sws[1] = P.sh_down_s;
    a.src = h; a.gsum = hsum; a.tiles = reinterpret_cast<const int4*>(tiles); a.ntiles = ntiles;
    a.dout = reinterpret_cast<uint16_t*>(dpart); a.H = H; a.I = I; a.E = E;
    return launch_mm<1>(a, (long)max_tiles * (H / 256), s);
}

}  // namespace glmmoe
