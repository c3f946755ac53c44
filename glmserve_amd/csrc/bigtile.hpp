// Work items of the large-group (128-row tile) expert kernels, shared by the
// W4A16 and FP8 variants.
//
// An item is (row tile, feature group): tiles come from the dispatch tile list
// ({expert, first grouped row, rows, -}); the feature group selects which
// slice of the output features the workgroup computes. Workgroups walk the
// items in rounds (item = round * grid + slot) and stage the next few items'
// headers and row -> token maps in an LDS table, so the streaming loop reads
// only LDS (a vector load in that loop would make the compiler drain the
// LDS-DMA queue with vmcnt(0)).
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace glmmoe {

constexpr int kBigTable = 3;              // items per table refill
constexpr int kBigTabInts = 4 + kBigRows; // {expert, row0, nrows, feature group} + row map

struct BigItem {
    int e, r0, nr, g;
    int hs;                    // 64-row item (a half tile): twice the features
    uint32_t tab;              // LDS address of the item's table entry
};

// Item k of the table at `table` (LDS); fields are wave-uniform (SGPRs).
__device__ __forceinline__ BigItem big_item(const char* table, int k) {
    const uint32_t base = lds_addr(table + k * kBigTabInts * 4);
    const uint4 hd = lds_bcast16(base);
    BigItem it;
    it.e = sgpr(hd.x);
    it.r0 = sgpr(hd.y);
    it.nr = sgpr(hd.z);
    it.g = sgpr(hd.w & 0xffffu);
    it.hs = sgpr(hd.w >> 16);
    it.tab = base;
    return it;
}

__device__ __forceinline__ uint32_t lds_read32(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1\n s_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr));
    return v;
}
__device__ __forceinline__ void lds_write32(uint32_t addr, float v) {
    asm volatile("ds_write_b32 %0, %1\n s_waitcnt lgkmcnt(0)" : : "v"(addr), "v"(v) : "memory");
}

// Item of workgroup b at round k. Workgroups are dispatched round-robin over
// the 8 XCDs (b % 8), each with its own L2; the items of one round are laid
// out so that each XCD takes a contiguous run of item ids -- the feature
// groups of the same row tile -- and the tile's activation rows are fetched
// into that XCD's L2 once instead of once per XCD.
__device__ __forceinline__ long big_item_id(long k) {
    const int nb = gridDim.x, b = blockIdx.x;
    const int lane_in_round = (nb % 8 == 0) ? (b % 8) * (nb / 8) + b / 8 : b;
    return k * nb + lane_in_round;
}

// Rounds that hold an item for this workgroup (ids at or past total are idle).
__device__ __forceinline__ long big_rounds(long total) {
    const long rounds = (total + gridDim.x - 1) / gridDim.x;
    if (rounds > 0 && big_item_id(rounds - 1) >= total) return rounds - 1;
    return rounds;
}

// Table rows for items k0 .. k0 + cnt - 1 of this workgroup. Row map entries:
// the token of each grouped row (GATHER, first projection) or the grouped row
// itself (second projection); rows past the tile's end repeat row 0.
template <bool GATHER>
__device__ __forceinline__ void big_fill_table(const int4* tiles, const int* rows_tok, int* table,
                                               long k0, int cnt, int nfg) {
    for (int i = threadIdx.x; i < cnt * kBigTabInts; i += blockDim.x) {
        const int k = i / kBigTabInts, f = i % kBigTabInts;
        const long item = big_item_id(k0 + k);
        const int4 tile = tiles[item / nfg];
        int v;
        if (f == 0) v = tile.x;
        else if (f == 1) v = tile.y;
        else if (f == 2) v = tile.z;
        else if (f == 3) v = (int)(item % nfg);
        else {
            const int row = f - 4;
            const int rr = row < tile.z ? row : 0;
            v = GATHER ? rows_tok[tile.y + rr] : tile.y + rr;
        }
        table[i] = v;
    }
}

// Expert-major item order (tile lists in expert order, every tile full-class):
// the items of expert e are ids [f nfg, (f + m) nfg) for its m tiles from tile
// f, and id f nfg + i is feature group i / m of tile f + i % m. So the m tiles
// of one (expert, feature group) are neighbours in the id order, run at the
// same time on one XCD and read the group's weights into its L2 once; the
// tile's nfg feature groups stay within m nfg neighbouring ids.
template <bool GATHER>
__device__ __forceinline__ void big_fill_table_em(const int4* tiles, const int* rows_tok, int* table,
                                                  long k0, int cnt, int nfg) {
    for (int i = threadIdx.x; i < cnt * kBigTabInts; i += blockDim.x) {
        const int k = i / kBigTabInts, f = i % kBigTabInts;
        const long item = big_item_id(k0 + k);
        const long t0 = item / nfg;
        const int w = tiles[t0].w;
        const int j = w & 0xffff, m = max(w >> 16, 1);
        const long first = t0 - j;
        const long local = item - first * nfg;
        const int4 tile = tiles[first + local % m];
        int v;
        if (f == 0) v = tile.x;
        else if (f == 1) v = tile.y;
        else if (f == 2) v = tile.z;
        else if (f == 3) v = (int)(local / m);
        else {
            const int row = f - 4;
            const int rr = row < tile.z ? row : 0;
            v = GATHER ? rows_tok[tile.y + rr] : tile.y + rr;
        }
        table[i] = v;
    }
}

// Items of a tile list with half tiles (W4A16 kernels): the first n128 tiles
// take nfg 128-row items each, the half tiles after them nfg / 2 64-row items
// (each twice as many features wide).
__device__ __forceinline__ long big2_total(int ntiles, int n128, int nfg) {
    return (long)n128 * nfg + (long)(ntiles - n128) * (nfg / 2);
}

__device__ __forceinline__ void big2_locate(long id, int n128, int nfg, int& tile, int& g, int& hs) {
    const long full = (long)n128 * nfg;
    if (id < full) {
        tile = (int)(id / nfg);
        g = (int)(id % nfg);
        hs = 0;
    } else {
        const long j = id - full;
        tile = n128 + (int)(j / (nfg / 2));
        g = (int)(j % (nfg / 2));
        hs = 1;
    }
}

template <bool GATHER>
__device__ __forceinline__ void big2_fill_table(const int4* tiles, const int* rows_tok, int* table,
                                                long k0, int cnt, int nfg, int n128) {
    for (int i = threadIdx.x; i < cnt * kBigTabInts; i += blockDim.x) {
        const int k = i / kBigTabInts, f = i % kBigTabInts;
        int ti, g, hs;
        big2_locate(big_item_id(k0 + k), n128, nfg, ti, g, hs);
        const int4 tile = tiles[ti];
        int v;
        if (f == 0) v = tile.x;
        else if (f == 1) v = tile.y;
        else if (f == 2) v = tile.z;
        else if (f == 3) v = g | (hs << 16);
        else {
            const int row = f - 4;
            const int rr = row < tile.z ? row : 0;
            v = GATHER ? rows_tok[tile.y + rr] : tile.y + rr;
        }
        table[i] = v;
    }
}

}  // namespace glmmoe
