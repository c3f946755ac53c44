// W4A16 experts, large-group regime (prefill and wide verify batches):
// grouped GEMM tiles of up to 128 grouped rows x 512 weight rows on fp16
// MFMA 32x32x16.
//
// Reference: the expert-major tensor-core path of the reference's GGUF MoE
// (cuda/qgemm.cu:1269-1356, emajor_mma_s8_kernel, used once n*topk reaches
// GLMSERVE_MMA_MOE_MIN_TS) and its W4A16 expert FFN semantics
// (cuda/moe_expert.cu:143-222).
//
// Work item = (row tile, feature group). A workgroup of 8 waves computes
// 128 rows x 512 weight rows: for gate/up 256 features (their gate rows and
// their up rows), for down 512 features. Wave w owns ALL 128 rows (4 row
// blocks of 32: the MFMA A operand, read from LDS) and 64 weight rows (2
// column blocks of 32: the B operand, decoded in registers): for gate/up 32
// gate rows and the 32 up rows of the same features, so SiLU(g) * u pairs
// in one lane; for down 64 features. Every A fragment feeds 2 MFMAs and
// every decoded B fragment 4.
//
// Operands are fp16. The weights decode straight to their dequantized value
// (c - 8) * s rounded once to fp16: with the int4 code c placed in mantissa
// bits 6-9 of 0x4800 (the fp16 of 8 + c / 2, exact), one packed fma
//   (8 + c / 2) * 2s - 24s = (c - 8) * s
// whose inputs 2s and 24s are exact in fp16 (s is a bf16 scale: 8
// significant bits) rounds only the result. So the accumulators need no
// per-group rescale and no offset correction: acc += A . B directly, fp32.
// The scales enter the decode multiplied by 2^kWPre (exact), so scales from
// 2^-(15 + kWPre) to 2729 * 2^-kWPre decode without fp16 subnormals or
// overflow; the epilogues undo the factor.
// Activations: gate/up reads x converted to fp16 with a per-row power-of-2
// scale (f16_rows_kernel below; exact for any finite bf16 row) and undoes the
// scale on its outputs; down reads the fp16 h this gate/up wrote. fp16 keeps
// 11 significant bits (bf16 keeps 8) but only 5 exponent bits, so h is stored
// with a power-of-2 exponent per row: the gate/up epilogue picks one per
// (row, 32 features) by a monotone rule of the block's largest |h|
// (h_exp_rule), h_rescale_kernel brings every block of a row to the row's
// smallest exponent (the rule of the row's largest |h|), and the down
// epilogue undoes it per row. Any finite h then reaches down in fp16 normal
// range: no overflow to inf, no row flushed to subnormals.
//
// Streams, per 128-K group g:
// - activations: 128 rows x 256 B (gathered by token for gate/up) global ->
//   LDS by buffer-load DMA into a 4-slot ring, issued 3 groups ahead. A row
//   occupies 272 B of its slot (16 B of padding), so the 16 rows of a
//   fragment read fall on 16 distinct bank groups and every fragment address
//   is the lane's base plus an immediate offset;
// - weights: each lane loads its own 2 x 32 B of int4 straight into
//   registers (a 2-deep ring; each half refilled as soon as its last step is
//   decoded, 1.5 groups ahead);
// - per batch of 8 groups: the bf16 scales of the workgroup's 32 tiles, one
//   DMA per wave into double buffers.
// One s_barrier per group, at its start, publishes slot g + 1 (every wave
// waited for its own DMAs of g + 1) and frees slot g - 1 for group g + 3.
// The DMAs and loads are issued one per K-step, so they overlap the MFMAs.
//
// Row blocks past a tile's last row skip their MFMAs and fragment reads: the
// dispatch lists full tiles first, then every expert's last tile of 33-64
// rows, then of at most 32 rows; a workgroup's items run class by class, each
// chunk through a pipeline specialized to its live row blocks (a run-time
// branch around an MFMA would make the compiler copy whole accumulators).
#include "common.hpp"
#include "bigtile.hpp"
#include "kernels.hpp"

namespace glmmoe {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

struct MmArgs {
    const uint8_t* wq[2];     // packed int4 tiles of the routed experts (gate, up) or (down, down)
    const uint16_t* ws[2];    // bf16 scales [rows/16][K/128][16]
    const uint8_t* swq[2];    // the shared expert's
    const uint16_t* sws[2];
    const uint16_t* src;      // fp16: xh [n, H] (gate/up, rows gathered by token) or h [R, I] (down)
    const float* rho;         // gate/up: per-token factor undoing xh's row scale
    const int4* tiles; const int* ntiles; const int* rows_tok;
    uint16_t* h;              // gate/up output: fp16 [R, I], row r scaled by 2^e(r)
    int8_t* hexp;             // [R, I / 32] exponents of h's 32-feature blocks (after
                              // h_rescale_kernel: every block of a row holds e(r))
    uint16_t* dout;           // down output: bf16 [R, H]
    // Split last round (gate/up): the items of a short last round run as two
    // K halves each; partials [item][half][wave][128][64] fp32, a ticket per
    // item (zero at launch). part null: no split.
    unsigned int* tick; float* part; int pcap;
    int H, I, E;
};

constexpr int kMmPartFloats = 8 * 128 * 64;   // one half item's accumulators
constexpr int kHExpNone = 127;                 // exponent of an all-zero block: no constraint

// Exponent e for a block whose largest |h| has fp32 bits m: 0 while
// 2^-6 <= |h| < 2^15 (fp16's normal range with 11 significant bits to spare
// below); outside that band the block's largest |h| * 2^e lands in
// [2^14, 2^15). Non-increasing in m, so the smallest e over a row's blocks is
// the rule of the row's largest |h|.
__device__ __forceinline__ int h_exp_rule(uint32_t m) {
    if (m == 0) return kHExpNone;
    const int e2 = (int)(m >> 23) - 127;   // inf / NaN: 128
    if (e2 >= 15 || e2 < -6) {
        const int e = 14 - e2;
        return e > 126 ? 126 : e;
    }
    return 0;
}

// Maximum of v over the 32 lanes of the wave's half that holds this lane.
__device__ __forceinline__ uint32_t max_half_wave(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));   // quad xor 1
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));   // quad xor 2
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xF, 0xF, false));  // row_ror 4
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false));  // row_ror 8
    v = max(v, (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401F));                    // lane xor 16
    return v;
}

namespace mm {
constexpr int kRowB = 272;                     // LDS bytes per activation row (256 + 16 padding)
constexpr int kSlot = 128 * kRowB;             // 34 KiB: 34 DMAs of 1 KiB
constexpr int kRing = 4;
constexpr int kSBuf = kRing * kSlot;           // 2 x 8 KiB: [tile 32][group 8][row 16] bf16
constexpr int kTab = kSBuf + 2 * 8192;
constexpr int kTabItems = 6;
constexpr int kRho = kTab + kTabItems * kBigTabInts * 4;   // [item][128] fp32 row factors
constexpr int kTotal = kRho + kTabItems * kBigRows * 4;
static_assert(kTotal <= 160 * 1024, "one workgroup's LDS");
constexpr int kBlk = 32 * kRowB;               // one 32-row block
}  // namespace mm

// Scale-buffer tile of lane column col in column block cb of wave w: the
// workgroup's 32 tiles per group are, for gate/up, gate tiles 16 g + 0..15
// then up tiles 16 g + 0..15; for down tiles 32 g + 0..31. Column block cb of
// wave w holds, for gate/up, matrix cb's tile 16 g + 2 w + col / 16; for down
// tile 32 g + 4 w + 2 cb + col / 16.
template <int NMAT>
__device__ __forceinline__ int mm_sbuf_tile(int wave, int cb, int col) {
    return NMAT == 2 ? 16 * cb + 2 * wave + (col >> 4) : 4 * wave + 2 * cb + (col >> 4);
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

// Stream state of one item.
//   act[i] (per lane): byte offset (in src) of this lane's 16 B of activation
//     DMA i at group 0; DMA d = wave + 8 i (i < 4) or 32 + (wave & 1) (i = 4;
//     waves 2-7 repeat DMAs 32 and 33 of waves 0, 1: same source, same LDS
//     bytes, so every wave waits for the same counts) fills slot bytes
//     1024 d + 16 lane = row p / 17, 16-B chunk p % 17 (p = 64 d + lane);
//     chunk 16 is padding (loads chunk 0 again);
//   wb[cb] (uniform): base of the wave's weight tiles of column block cb; a
//     lane adds the item-invariant MmLane::w (its 32 B of int4: K positions
//     64 h .. 64 h + 63 of weight row col % 16 of its tile);
//   sb (uniform): base of the scales of the workgroup's 32 tiles (as the
//     wave sees them: the wave's 4 tiles share one matrix); a lane adds
//     MmLane::s.
// Only act needs vector registers: the item's other addresses are scalar.
struct MmPtrs {
    uint32_t act[5];
    const uint8_t* wb[2];
    const uint16_t* sb;
};
struct MmLane {
    uint32_t w, s;
};

// The item-invariant lane offsets:
//   gate/up: weight tile 16 g + (2 w + col / 16), scale tile 16 g + (4 w + lane / 16) % 16;
//   down:    weight tile 32 g + 2 cb + (4 w + col / 16), scale tile 32 g + (4 w + lane / 16).
template <int NMAT>
__device__ __forceinline__ MmLane mm_lane(int KG, int wave, int lane) {
    const int col = lane & 31, h = lane >> 5;
    const int tl = NMAT == 2 ? 2 * wave + (col >> 4) : 4 * wave + (col >> 4);
    const int ts = NMAT == 2 ? (4 * wave + (lane >> 4)) & 15 : 4 * wave + (lane >> 4);
    MmLane l;
    l.w = (uint32_t)tl * KG * 1024 + (col & 15) * 16 + h * 512;
    l.s = ((uint32_t)ts * KG * 16 + (lane & 15) * 8) * 2u;
    return l;
}

// act[i] of the item whose table entry is at LDS address tab.
__device__ __forceinline__ uint32_t mm_act(uint32_t tab, int K, int wave, int lane, int i) {
    const int d = i < 4 ? wave + 8 * i : 32 + (wave & 1);
    const int pos = 64 * d + lane;
    const int row = pos / 17, c = pos % 17;
    return lds_read32(tab + 16 + row * 4) * (uint32_t)(K * 2) + (uint32_t)((c & 15) * 16);
}

// ACT false: the scalar addresses only (act left zero).
template <int NMAT, bool ACT = true>
__device__ __forceinline__ MmPtrs mm_ptrs(const MmArgs& a, const BigItem& it, int K, int KG, int wave,
                                          int lane) {
    MmPtrs p;
    // A half item (hs 1 or 2: the first or second half of K) starts its
    // streams at batch kb0.
    const int kb0 = (it.hs & 3) == 2 ? K / 2048 : 0;
#pragma unroll
    for (int i = 0; i < 5; ++i) p.act[i] = ACT ? mm_act(it.tab, K, wave, lane, i) + (uint32_t)kb0 * 2048u : 0u;
    const int frows = NMAT == 2 ? a.I : a.H;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        const int m = NMAT == 2 ? cb : 0;
        const int fb = NMAT == 2 ? 16 * it.g : 32 * it.g + 2 * cb;
        p.wb[cb] = mm_wbase<NMAT>(a, it.e, m, frows, KG) + (size_t)fb * KG * 1024 + (size_t)kb0 * 8192;
    }
    {
        const int m = NMAT == 2 ? (wave >> 2) : 0;
        const int fb = NMAT == 2 ? 16 * it.g : 32 * it.g;
        p.sb = mm_sbase<NMAT>(a, it.e, m, frows, KG) + (size_t)fb * KG * 16 + (size_t)kb0 * 128;
    }
    return p;
}

// Fragments of NB row blocks, OFF past addr, block b at OFF + b * kBlk.
template <int NB, int OFF>
__device__ __forceinline__ void lds_frags(uint32_t addr, u32x4 (&a)[4]) {
    if constexpr (NB == 1) {
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(a[0]) : "v"(addr), "n"(OFF));
    } else if constexpr (NB == 2) {
        asm volatile("ds_read_b128 %0, %2 offset:%3\n ds_read_b128 %1, %2 offset:%4"
                     : "=&v"(a[0]), "=&v"(a[1])
                     : "v"(addr), "n"(OFF), "n"(OFF + mm::kBlk));
    } else {
        asm volatile("ds_read_b128 %0, %4 offset:%5\n ds_read_b128 %1, %4 offset:%6\n"
                     " ds_read_b128 %2, %4 offset:%7\n ds_read_b128 %3, %4 offset:%8"
                     : "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(a[3])
                     : "v"(addr), "n"(OFF), "n"(OFF + mm::kBlk), "n"(OFF + 2 * mm::kBlk),
                       "n"(OFF + 3 * mm::kBlk));
    }
}
// Waits until at most N LDS operations are pending; the fragment registers
// (and extra registers written by pending reads) are operands, so nothing
// reads them before the data has arrived.
template <int N, int NB>
__device__ __forceinline__ void lgkm_frags(u32x4 (&a)[4]) {
    if constexpr (NB == 1) asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(a[0]) : "n"(N));
    else if constexpr (NB == 2) asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a[0]), "+v"(a[1]) : "n"(N));
    else
        asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]) : "n"(N));
}

__device__ __forceinline__ void dma_buf16(__amdgpu_buffer_rsrc_t r, uint32_t lds_dst, uint32_t voff,
                                          uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)(uintptr_t)lds_dst, 16, voff, soff, 0, 0);
}

// One lane's 16 B of weights: buffer load at base + voff + soff (compiler
// visible: the compiler waits for it before any use or copy of dst). The
// weights are read once: streaming (non-temporal) cache policy.
__device__ __forceinline__ void w_load(u32x4& dst, const uint8_t* base, uint32_t voff, uint32_t soff) {
    dst = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(mm_rsrc(base), voff, soff, 2));
}

__device__ __forceinline__ f32x16 mfma16(u32x4 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                  c, 0, 0, 0);
}

// The fp16 decode constants as opaque registers (mask of mantissa bits 6-9
// of both halves, the fp16 pattern of 8.0 in both halves): with literal
// operands the compiler splits v_and_or_b32.
struct DqF16 {
    uint32_t mask, bias;
};
__device__ __forceinline__ DqF16 dq_f16_const() {
    DqF16 c;
    asm volatile("v_mov_b32 %0, 0x03c003c0\n v_mov_b32 %1, 0x48004800" : "=v"(c.mask), "=v"(c.bias));
    return c;
}

// Dequantized fp16 weights of one packed dword (8 K positions; position 2j
// in nibble j, 2j + 1 in nibble j + 4): fp16x2 j = ((c - 8) * s) of positions
// 2j, 2j + 1. s2 = {2s, 2s}, s24 = {-24s, -24s}.
__device__ __forceinline__ bf16x8 dq_f16(uint32_t w, const DqF16& k, f16x2 s2, f16x2 s24) {
    const uint32_t v0 = ((w << 6) & k.mask) | k.bias;
    const uint32_t v1 = ((w << 2) & k.mask) | k.bias;
    const uint32_t v2 = ((w >> 2) & k.mask) | k.bias;
    const uint32_t v3 = ((w >> 6) & k.mask) | k.bias;
    u32x4 r;
    r.x = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2, v0), s2, s24));
    r.y = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2, v1), s2, s24));
    r.z = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2, v2), s2, s24));
    r.w = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2, v3), s2, s24));
    return __builtin_bit_cast(bf16x8, r);
}

// {2s, 2s} and {-24s, -24s} times 2^kWPre in fp16 from a bf16 scale pattern
// (exact for scales in 2^-(15 + kWPre) .. 2729 * 2^-kWPre).
__device__ __forceinline__ void scale_pair(uint32_t sbits, f16x2& s2, f16x2& s24) {
    const float s = bf16_to_f32(sbits & 0xffffu);
    constexpr float kPre = (float)(1 << kWPre);
    const _Float16 a = (_Float16)((2.0f * kPre) * s), b = (_Float16)((-24.0f * kPre) * s);
    s2 = f16x2{a, a};
    s24 = f16x2{b, b};
}

// Stores an item's outputs through stg, 1 KiB of LDS private to the wave: the
// accumulator layout gives a lane one feature of 4 consecutive rows, so each
// round writes a block of rows x features to stg (2-byte writes) and reads it
// back as 16 contiguous bytes of one row per lane, stored with one 16-B
// global store (8x fewer stores than element-wise: stores count in the same
// vmcnt as the stream's prefetches, so fewer of them means a shorter drain).
// rho (gate/up): the item's row factors in LDS.
template <int NMAT>
__device__ __forceinline__ void mm_epilogue(const MmArgs& a, const BigItem& cur, uint32_t rho, uint32_t stg,
                                            int wave, int lane, f32x16 (&acc)[4][2]) {
    // Laundered lane index: keeps the per-row addresses below from being
    // hoisted out of the streaming loop (they would stay live and spill).
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int col = ln & 31, h = ln >> 5;
    if constexpr (NMAT == 2) {
        // h = silu(g) * u of this lane's feature (rows' scale undone first);
        // a round is 16 rows x this wave's 32 features of fp16, each row
        // scaled by 2^e of its largest |h| among those features.
        uint16_t* hbase = a.h + (size_t)cur.r0 * a.I + cur.g * 256 + wave * 32 + (ln & 3) * 8;
        int8_t* ebase = a.hexp + (size_t)cur.r0 * (a.I / 32) + cur.g * 8 + wave;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            float rr[16];   // row factors of the lane's 16 rows of block rb
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 v = lds_bcast16(rho + (uint32_t)((rb * 32 + 8 * q + 4 * h) * 4));
                rr[4 * q] = __uint_as_float(v.x);
                rr[4 * q + 1] = __uint_as_float(v.y);
                rr[4 * q + 2] = __uint_as_float(v.z);
                rr[4 * q + 3] = __uint_as_float(v.w);
            }
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                float hf[8];
                uint32_t mx[8];
#pragma unroll
                for (int ii = 0; ii < 8; ++ii) {
                    const int i = half * 8 + ii;
                    const float gt = acc[rb][0][i] * rr[i], up = acc[rb][1][i] * rr[i];
                    hf[ii] = silu_fast(gt) * up;
                    mx[ii] = max_half_wave(__float_as_uint(hf[ii]) & 0x7fffffffu);
                }
#pragma unroll
                for (int ii = 0; ii < 8; ++ii) {
                    const int e = h_exp_rule(mx[ii]);
                    const float hs = __builtin_ldexpf(hf[ii], e == kHExpNone ? 0 : e);
                    const uint16_t hv = __builtin_bit_cast(uint16_t, (_Float16)hs);
                    const int rl = 8 * (ii >> 2) + 4 * h + (ii & 3);   // row within the round
                    asm volatile("ds_write_b16 %0, %1" : : "v"(stg + (uint32_t)(rl * 64 + col * 2)), "v"((uint32_t)hv)
                                 : "memory");
                    const int row = rb * 32 + half * 16 + rl;
                    if (col == 0 && row < cur.nr) ebase[(size_t)row * (a.I / 32)] = (int8_t)e;
                }
                const uint4 v = lds_bcast16(stg + (uint32_t)(ln * 16));
                const int row = rb * 32 + half * 16 + (ln >> 2);
                if (row < cur.nr) *reinterpret_cast<uint4*>(hbase + (size_t)row * a.I) = v;
            }
        }
    } else {
        // Per-row expert outputs as bf16 (the combine adds them in fp32), h's
        // row exponent and the weight factor undone (rho: the rows' factors);
        // a round is 8 rows x this wave's 64 features.
        uint16_t* dbase = a.dout + (size_t)cur.r0 * a.H + cur.g * 512 + wave * 64 + (ln & 7) * 8;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 fv = lds_bcast16(rho + (uint32_t)((rb * 32 + 8 * q + 4 * h) * 4));
                const float rf[4] = {__uint_as_float(fv.x), __uint_as_float(fv.y), __uint_as_float(fv.z),
                                     __uint_as_float(fv.w)};
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t bv = pack_bf16x2(acc[rb][cb][4 * q + e] * rf[e], 0.0f) & 0xffffu;
                        asm volatile("ds_write_b16 %0, %1"
                                     : : "v"(stg + (uint32_t)((4 * h + e) * 128 + (32 * cb + col) * 2)), "v"(bv)
                                     : "memory");
                    }
                const uint4 v = lds_bcast16(stg + (uint32_t)(ln * 16));
                const int row = rb * 32 + 8 * q + (ln >> 3);
                if (row < cur.nr) *reinterpret_cast<uint4*>(dbase + (size_t)row * a.H) = v;
            }
    }
}

template <int NMAT>
__global__ __launch_bounds__(512) void w4_mm_kernel(MmArgs a) {
    extern __shared__ __align__(16) char lds[];
    const DqF16 dqc = dq_f16_const();
    int* table = reinterpret_cast<int*>(lds + mm::kTab);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 31, h = lane >> 5;
    const int K = NMAT == 2 ? a.H : a.I;
    const int KG = K / 128;          // a multiple of 8 (checked by the launcher)
    const int NB = KG / 8;           // batches per item
    const int nfg = NMAT == 2 ? a.I / 256 : a.H / 512;
    // Tile classes by rows: more than 64, 33-64, at most 32 rows: 4, 2 and 1
    // live 32-row blocks (the dispatch lists them in that order, so a
    // workgroup's items run class by class in few chunks).
    const int nt = a.ntiles[0];
    // Items round-robin over the workgroups; a short last round (at most
    // half the workgroups busy) runs as two K halves per item on two
    // neighbouring workgroups, so it takes half as long.
    const long total = (long)nt * nfg;
    const int nb = gridDim.x;
    const long R = (total + nb - 1) / nb;
    const long rem = total - (R - 1) * nb;
    const bool split = NMAT == 2 && a.part != nullptr && R >= 1 && 2 * rem <= nb && rem <= a.pcap &&
                       rem <= kTailTicks && NB % 2 == 0;
    const int lir = (nb % 8 == 0) ? (blockIdx.x % 8) * (nb / 8) + blockIdx.x / 8 : blockIdx.x;   // big_item_id's slot
    const long nitems = split ? (R - 1) + (lir < 2 * rem ? 1 : 0) : big_rounds(total);
    // Item id of round k and its table tag: 0 whole, 1 / 2 first / second
    // half, with the half item's index (for its ticket and partials) above.
    auto ident = [&](long k, int& tag) -> long {
        if (split && k == R - 1) {
            tag = (1 + (lir & 1)) | ((lir >> 1) << 2);
            return (R - 1) * nb + (lir >> 1);
        }
        tag = 0;
        return big_item_id(k);
    };
    const uint32_t ring = lds_addr(lds);
    // Lane's fragment address at step 0 of row block 0 in slot 0: row col,
    // 16-B chunk 8 h; step s adds 16 s, row block rb 8704 rb, slot q 34 KiB q.
    const uint32_t xa0 = ring + (uint32_t)(col * mm::kRowB + h * 128);
    // Lane's scale of column block 0 in scale buffer 0 at group 0; column
    // block 1's is kSt1 bytes further.
    const uint32_t sa0 = lds_addr(lds + mm::kSBuf) +
                         (uint32_t)(mm_sbuf_tile<NMAT>(wave, 0, col) * 256 + (col & 15) * 2);
    constexpr int kSt1 = NMAT == 2 ? 16 * 256 : 2 * 256;
    const __amdgpu_buffer_rsrc_t rsrc_src = mm_rsrc(a.src);
    const MmLane ml = mm_lane<NMAT>(KG, wave, lane);

    auto cls_of = [&](long k) {
        int tag;
        const int nr = a.tiles[ident(k, tag) / nfg].z;
        return (nr > 64 ? 4 : nr > 32 ? 2 : 1) + (tag ? 8 : 0);
    };
    // One chunk (at most kTabItems items of one class): table, prologue,
    // stream, drain. The accumulators live only inside it.
    auto run_chunk = [&](auto NRB_, long k0, int cnt, bool halves) {
        constexpr int NRB = decltype(NRB_)::value;
        // Table rows (big_fill_table's layout; the tag in the high bits of
        // the feature-group word).
        for (int i = threadIdx.x; i < cnt * kBigTabInts; i += blockDim.x) {
            const int k = i / kBigTabInts, f = i % kBigTabInts;
            int tag;
            const long id = ident(k0 + k, tag);
            const int4 tile = a.tiles[id / nfg];
            int v;
            if (f == 0) v = tile.x;
            else if (f == 1) v = tile.y;
            else if (f == 2) v = tile.z;
            else if (f == 3) v = (int)(id % nfg) | (tag << 16);
            else {
                const int row = f - 4;
                const int rr = row < tile.z ? row : 0;
                v = NMAT == 2 ? a.rows_tok[tile.y + rr] : tile.y + rr;
            }
            table[i] = v;
        }
        __syncthreads();
        {
            // Row factors: gate/up x's row scale and the weight factor
            // (f16_rows_kernel folds both into rho); down h's row exponent
            // and the weight factor.
            float* rho = reinterpret_cast<float*>(lds + mm::kRho);
            for (int i = threadIdx.x; i < cnt * kBigRows; i += blockDim.x) {
                const int row = table[(i / kBigRows) * kBigTabInts + 4 + (i % kBigRows)];
                if constexpr (NMAT == 2) rho[i] = a.rho[row];
                else rho[i] = __builtin_ldexpf(1.0f, -((int)a.hexp[(size_t)row * (a.I / 32)] + kWPre));
            }
            __syncthreads();
        }
        const int NBi = halves ? NB / 2 : NB;   // batches per item
        const int NBt = cnt * NBi;              // batches of this chunk
        auto item = [&](int k) { return big_item(lds + mm::kTab, k < cnt ? k : cnt - 1); };

        // Stream state of the item of the current batch (pc) and of the next
        // item (pn; past the chunk's end the last item again: those loads
        // land in buffers nobody reads). In the last batch of an item the
        // activation stream (3 groups ahead) and the weight stream (2 ahead)
        // cross into the next item at fixed group positions.
        // The next item's act offsets are read from its table entry when
        // needed (5 fewer registers held through the stream).
        MmPtrs pc = mm_ptrs<NMAT>(a, item(0), K, KG, wave, lane);
        MmPtrs pn = mm_ptrs<NMAT, false>(a, item(1), K, KG, wave, lane);
        auto next_tab = [&](int k) {
            return lds_addr(lds + mm::kTab) + (uint32_t)((k + 1 < cnt ? k + 1 : cnt - 1) * kBigTabInts * 4);
        };
        u32x4 W[2][2][2];   // [ring][column block][lo / hi 16 B]
        auto issue_w = [&](const MmPtrs& p, int k, int r, int half) {
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
                w_load(W[r][cb][half], p.wb[cb], ml.w, (uint32_t)(k * 1024 + half * 256));
        };
        auto issue_act = [&](uint32_t act, int k, int gslot, int i) {
            const uint32_t dst = ring + (uint32_t)((gslot & 3) * mm::kSlot);
            const int d = i < 4 ? wave + 8 * i : 32 + (wave & 1);
            dma_buf16(rsrc_src, dst + (uint32_t)(d * 1024), act, (uint32_t)k * 256u);
        };
        auto issue_scales = [&](const uint16_t* sb, int kb, int parity) {
            dma_buf16(mm_rsrc(sb), lds_addr(lds + mm::kSBuf + parity * 8192 + wave * 1024), ml.s,
                      (uint32_t)kb * 256u);
        };

        // Prologue: scales of batch 0, activation groups 0-2, weights 0-1.
        issue_scales(pc.sb, 0, 0);
#pragma unroll
        for (int g0 = 0; g0 < 3; ++g0)
#pragma unroll
            for (int i = 0; i < 5; ++i) issue_act(pc.act[i], g0, g0, i);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            issue_w(pc, r, r, 0);
            issue_w(pc, r, r, 1);
        }
        wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();

        f32x16 acc[4][2];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) acc[rb][0] = acc[rb][1] = f32x16{};
        // Scales of group 0 and the decoded B of its step 0.
        f16x2 s2[2], s24[2];
        scale_pair(lds_read_u16(sa0), s2[0], s24[0]);
        scale_pair(lds_read_u16(sa0 + kSt1), s2[1], s24[1]);
        bf16x8 Bd[2][2];   // [parity][column block]
        Bd[0][0] = dq_f16(W[0][0][0][0], dqc, s2[0], s24[0]);
        Bd[0][1] = dq_f16(W[0][1][0][0], dqc, s2[1], s24[1]);
        // Fragments of step 0 of group 0.
        u32x4 A[2][4];
        lds_frags<NRB, 0>(xa0, A[0]);
        int ib = 0, kb = 0;   // item and batch-in-item of the current batch

        for (int b = 0; b < NBt; ++b) {
            const bool last = kb == NBi - 1;
            static_for<8>([&](auto J) {
                constexpr int j = decltype(J)::value;
                // ---- group start: publish slot g + 1, free slot g - 1. Pending
                // before the wait: this wave's DMAs of g + 1 (issued in g - 2,
                // the last at step 4) and what followed them in g - 2: the
                // scale DMA if it opened a batch (step 5) and the high weights
                // (step 6, 2 loads); then all of g - 1's issue (5 DMAs, 4 weight
                // loads, maybe the scale DMA).
                {
                    constexpr int n2 = (((j + 6) & 7) == 0 ? 1 : 0) + 2;
                    constexpr int n1 = 9 + (((j + 7) & 7) == 0 ? 1 : 0);
                    wait_vmcnt<n2 + n1>();
                }
                __builtin_amdgcn_s_barrier();
                // Fragment base of slot g and g + 1 (opaque scalar offsets).
                uint32_t so = (uint32_t)((j & 3) * mm::kSlot), nso = (uint32_t)(((j + 1) & 3) * mm::kSlot);
                asm volatile("" : "+s"(so), "+s"(nso));
                const uint32_t xg = xa0 + so;
                // Stream sources: activations of group g + 3, weights of group
                // g + 2 (this item's or, late in the item's last batch, the next
                // item's: selects, no branches).
                int ka = 8 * kb + j + 3;
                if constexpr (j >= 5) ka = last ? j - 5 : ka;
                MmPtrs pw = pc;
                int kw = 8 * kb + j + 2;
                if constexpr (j >= 6) {
                    pw.wb[0] = last ? pn.wb[0] : pc.wb[0];
                    pw.wb[1] = last ? pn.wb[1] : pc.wb[1];
                    kw = last ? j - 6 : kw;
                }
                uint32_t nsr0 = 0, nsr1 = 0;   // scales of g + 1
                static_for<8>([&](auto S_) {
                    constexpr int s = decltype(S_)::value;
                    constexpr int cbuf = s & 1, nbuf = cbuf ^ 1;
                    // Fragments of step s + 1 (or step 0 of g + 1).
                    if constexpr (s < 7) lds_frags<NRB, 16 * (s + 1)>(xg, A[nbuf]);
                    else lds_frags<NRB, 0>(xa0 + nso, A[nbuf]);
                    if constexpr (s == 4) {
                        // Scales of g + 1 (after a batch's last group: the next
                        // batch's buffer, written in this batch's first group).
                        const uint32_t sb = sa0 + (uint32_t)((j == 7 ? ((b + 1) & 1) : (b & 1)) * 8192 +
                                                             ((j + 1) & 7) * 32);
                        asm volatile("ds_read_u16 %0, %2\n ds_read_u16 %1, %2 offset:%3"
                                     : "=&v"(nsr0), "=&v"(nsr1)
                                     : "v"(sb), "n"(kSt1));
                    }
                    // Each row block's MFMAs start as soon as its fragment is
                    // in (LDS reads complete in order; pending behind it: the
                    // step's later fragments, step s + 1's and, at step 4,
                    // the 2 scale reads).
                    static_for<NRB>([&](auto R_) {
                        constexpr int rb = decltype(R_)::value;
                        constexpr int n = (s == 4 ? 2 : 0) + NRB + (NRB - 1 - rb);
                        if constexpr (s == 5 && rb == NRB - 1)
                            asm volatile("s_waitcnt lgkmcnt(%3)" : "+v"(A[cbuf][rb]), "+v"(nsr0), "+v"(nsr1) : "n"(n));
                        else
                            asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(A[cbuf][rb]) : "n"(n));
                        acc[rb][0] = mfma16(A[cbuf][rb], Bd[cbuf][0], acc[rb][0]);
                        acc[rb][1] = mfma16(A[cbuf][rb], Bd[cbuf][1], acc[rb][1]);
                    });
                    // Decode step s + 1 (or step 0 of g + 1 with its scales).
                    if constexpr (s < 7) {
#pragma unroll
                        for (int cb = 0; cb < 2; ++cb)
                            Bd[nbuf][cb] = dq_f16(W[j & 1][cb][(s + 1) >> 2][(s + 1) & 3], dqc, s2[cb], s24[cb]);
                    } else {
                        scale_pair(nsr0, s2[0], s24[0]);
                        scale_pair(nsr1, s2[1], s24[1]);
#pragma unroll
                        for (int cb = 0; cb < 2; ++cb)
                            Bd[nbuf][cb] = dq_f16(W[(j + 1) & 1][cb][0][0], dqc, s2[cb], s24[cb]);
                    }
                    // Issue one stream piece per step.
                    if constexpr (s <= 4) {
                        uint32_t act = pc.act[s];
                        if constexpr (j >= 5) act = last ? mm_act(next_tab(ib), K, wave, lane, s) : act;
                        issue_act(act, ka, j + 3, s);
                    }
                    if constexpr (s == 2) issue_w(pw, kw, j & 1, 0);    // low halves of g decoded
                    if constexpr (s == 5 && j == 0)
                        issue_scales(last ? pn.sb : pc.sb, last ? 0 : kb + 1, (b + 1) & 1);
                    if constexpr (s == 6) issue_w(pw, kw, j & 1, 1);    // high halves of g decoded
                });
            });
            if (last) {
                // Item done: store it. The next group's first fragments are in
                // flight in A[0]; wait for them first.
                lgkm_frags<0, NRB>(A[0]);
                // Staging for the stores: this batch's scale buffer, read for
                // the last time in this batch's group 6 (the next batch's scale
                // DMA into it is issued after the next group-start barrier).
                bool store = true;
                if constexpr (NMAT == 2) {
                    if (halves) {
                        // Half item: store the partials, take the item's
                        // ticket; the second to arrive adds the other half
                        // (a + b, the same sum either way) and stores.
                        const int tag = item(ib).hs, half = (tag & 3) - 1, pi = tag >> 2;
                        float* dst = a.part + ((size_t)(pi * 2 + half) * 8 + wave) * 8192 + lane;
#pragma unroll
                        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                                for (int i = 0; i < 16; ++i) st_dev(dst + ((rb * 2 + cb) * 16 + i) * 64, acc[rb][cb][i]);
                        drain_vm();
                        __syncthreads();
                        int* flag = table + (mm::kTabItems - 1) * kBigTabInts;
                        if (threadIdx.x == 0) *flag = ticket_dev(&a.tick[pi]) == 1u ? 1 : 0;
                        __syncthreads();
                        store = *flag != 0;
                        __syncthreads();
                        if (store) {
                            const float* src = a.part + ((size_t)(pi * 2 + (1 - half)) * 8 + wave) * 8192 + lane;
#pragma unroll
                            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                                    for (int i = 0; i < 16; ++i)
                                        acc[rb][cb][i] = acc[rb][cb][i] + ld_dev(src + ((rb * 2 + cb) * 16 + i) * 64);
                        }
                    }
                }
                if (store)
                    mm_epilogue<NMAT>(a, item(ib), lds_addr(lds + mm::kRho + ib * kBigRows * 4),
                                      lds_addr(lds + mm::kSBuf + (b & 1) * 8192 + wave * 1024), wave, lane, acc);
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) acc[rb][0] = acc[rb][1] = f32x16{};
                ++ib;
                kb = 0;
                pc = mm_ptrs<NMAT>(a, item(ib), K, KG, wave, lane);
                pn = mm_ptrs<NMAT, false>(a, item(ib + 1), K, KG, wave, lane);
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
        while (cnt < mm::kTabItems - 1 && k0 + cnt < nitems && cls_of(k0 + cnt) == cls) ++cnt;
        const bool halves = cls >= 8;
        if ((cls & 7) == 4) run_chunk(std::integral_constant<int, 4>{}, k0, cnt, halves);
        else if ((cls & 7) == 2) run_chunk(std::integral_constant<int, 2>{}, k0, cnt, halves);
        else run_chunk(std::integral_constant<int, 1>{}, k0, cnt, halves);
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

// x (bf16) -> fp16 with a power-of-2 scale per row so the row's largest
// magnitude lies in [2^14, 2^15): exact for every finite bf16 row down to
// 2^-10 of the row maximum (bf16's 8 significant bits fit fp16's 11; smaller
// elements round to fp16's subnormal steps). rho[t] = the inverse factor
// times 2^-kWPre, applied to the row's outputs. One wave per row.
__global__ __launch_bounds__(256) void f16_rows_kernel(const uint16_t* __restrict__ x, int n, int H,
                                                      uint16_t* __restrict__ xh, float* __restrict__ rho) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= n) return;
    const uint16_t* xr = x + (size_t)t * H;
    uint32_t amax = 0;   // bf16 magnitudes compare as integers
    for (int i = lane * 8; i < H; i += 512) {
        const uint4 v = *reinterpret_cast<const uint4*>(xr + i);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            amax = max(amax, w[q] & 0x7fffu);
            amax = max(amax, (w[q] >> 16) & 0x7fffu);
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = max(amax, (uint32_t)__shfl_xor((int)amax, off));
    // Exponent of the row maximum (bf16 exponent field); all-zero rows use 0.
    const int e = amax >= 0x0080u ? (int)(amax >> 7) - 127 : 0;
    int k = 14 - e;                       // max * 2^k in [2^14, 2^15)
    k = k > 100 ? 100 : (k < -100 ? -100 : k);
    const float scale = __builtin_ldexpf(1.0f, k);
    if (lane == 0) rho[t] = __builtin_ldexpf(1.0f, -k - kWPre);   // also undoes the weights' factor
    uint16_t* yr = xh + (size_t)t * H;
    for (int i = lane * 8; i < H; i += 512) {
        const uint4 v = *reinterpret_cast<const uint4*>(xr + i);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const _Float16 lo = (_Float16)(bf16_to_f32(w[q] & 0xffffu) * scale);
            const _Float16 hi = (_Float16)(bf16_to_f32(w[q] >> 16) * scale);
            o[q] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
        }
        *reinterpret_cast<uint4*>(yr + i) = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// Brings every 32-feature block of an h row to the row's smallest block
// exponent (h_exp_rule is non-increasing, so that is the rule of the row's
// largest |h|): blocks with a larger exponent are multiplied by 2^(e_row - e)
// (exact unless the result is an fp16 subnormal, i.e. below 2^-24 of the
// row's largest |h| once scaled); every block byte then holds e_row. One
// thread per row reads the row's I / 32 exponent bytes (consecutive rows:
// coalesced 16-B loads); rows whose blocks already agree (every row whose |h|
// stays in the band) are only read.
__global__ __launch_bounds__(256) void h_rescale_kernel(uint16_t* __restrict__ h, int8_t* __restrict__ hexp, int R,
                                                       int I) {
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r >= R) return;
    const int nb = I / 32;   // a multiple of 16 (I % 1024 == 0)
    uint4* er = reinterpret_cast<uint4*>(hexp + (size_t)r * nb);
    int emin = kHExpNone, emax = -128;
    for (int v = 0; v < nb / 16; ++v) {
        const uint4 q = er[v];
        const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int e = (int)(int8_t)(d[j >> 2] >> (8 * (j & 3)));
            emin = min(emin, e);
            emax = max(emax, e);
        }
    }
    if (emin == emax) return;
    int8_t* eb = hexp + (size_t)r * nb;
    for (int b = 0; b < nb; ++b) {
        const int e = eb[b];
        if (e == emin) continue;
        uint4* p = reinterpret_cast<uint4*>(h + (size_t)r * I + b * 32);
        for (int q = 0; q < 4; ++q) {
            const uint4 v = p[q];
            uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float lo = __builtin_ldexpf((float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] & 0xffffu)),
                                                  emin - e);
                const float hi = __builtin_ldexpf((float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] >> 16)),
                                                  emin - e);
                w[j] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
                       ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
            }
            p[q] = make_uint4(w[0], w[1], w[2], w[3]);
        }
        eb[b] = (int8_t)emin;
    }
}

bool big_w4_shape_ok(int H, int I) { return H % 1024 == 0 && I % 1024 == 0; }

// scratch: the dpart region (free until the down projection, scratch_bytes):
// xh [n, H] fp16, rho [n] fp32, then the split last round's partials; tick:
// its tickets (kTailTicks, zero at launch).
int launch_gate_up_big(const ExpertPtrs& P, const uint16_t* x, int n, const int* tiles,
                       const int* ntiles, int max_tiles, const int* rows_tok, uint16_t* h,
                       int8_t* hexp, void* scratch, size_t scratch_bytes, unsigned int* tick, int H,
                       int I, int E, hipStream_t s, bool x16_ready) {
    if (!big_w4_shape_ok(H, I)) return -2;
    uint16_t* xh = reinterpret_cast<uint16_t*>(scratch);
    float* rho = reinterpret_cast<float*>(xh + (size_t)n * H);
    if (!x16_ready) {
        hipLaunchKernelGGL(f16_rows_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, x, n, H, xh, rho);
        if (hipGetLastError() != hipSuccess) return -4;
    }
    MmArgs a{};
    a.wq[0] = P.gate_q; a.ws[0] = P.gate_s; a.wq[1] = P.up_q; a.ws[1] = P.up_s;
    a.swq[0] = P.sh_gate_q; a.sws[0] = P.sh_gate_s; a.swq[1] = P.sh_up_q; a.sws[1] = P.sh_up_s;
    a.src = xh; a.rho = rho; a.tiles = reinterpret_cast<const int4*>(tiles); a.ntiles = ntiles;
    a.rows_tok = rows_tok; a.h = h; a.hexp = hexp; a.H = H; a.I = I; a.E = E;
    // The split last round's partials after xh and rho (two halves per item).
    const size_t off = ((size_t)n * H * 2 + (size_t)n * 4 + 255) / 256 * 256;
    if (tick && scratch_bytes > off) {
        const size_t cap = (scratch_bytes - off) / ((size_t)2 * kMmPartFloats * 4);
        a.tick = tick;
        a.part = reinterpret_cast<float*>(reinterpret_cast<char*>(scratch) + off);
        a.pcap = (int)(cap < (size_t)kTailTicks ? cap : (size_t)kTailTicks);
    }
    return launch_mm<2>(a, (long)max_tiles * (I / 256), s);
}

int launch_down_big(const ExpertPtrs& P, uint16_t* h, int8_t* hexp, int R, const int* tiles,
                    const int* ntiles, int max_tiles, float* dpart, int H, int I, int E,
                    hipStream_t s) {
    if (!big_w4_shape_ok(H, I)) return -2;
    hipLaunchKernelGGL(h_rescale_kernel, dim3((unsigned)((R + 255) / 256)), dim3(256), 0, s, h, hexp, R, I);
    if (hipGetLastError() != hipSuccess) return -4;
    MmArgs a{};
    a.wq[0] = P.down_q; a.ws[0] = P.down_s; a.wq[1] = P.down_q; a.ws[1] = P.down_s;
    a.swq[0] = P.sh_down_q; a.sws[0] = P.sh_down_s; a.swq[1] = P.sh_down_q; a.sws[1] = P.sh_down_s;
    a.src = h; a.hexp = hexp; a.tiles = reinterpret_cast<const int4*>(tiles); a.ntiles = ntiles;
    a.dout = reinterpret_cast<uint16_t*>(dpart); a.H = H; a.I = I; a.E = E;
    return launch_mm<1>(a, (long)max_tiles * (H / 512), s);
}

}  // namespace glmmoe
