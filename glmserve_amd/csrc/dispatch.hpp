// Dispatch body shared by the stand-alone dispatch kernel and the fused
// small-batch routing kernel: expert histogram, prefix scan and a stable
// permute that groups the (token, slot) rows by expert, plus the inverse map
// and the tile list the grouped expert GEMMs walk.
//
// Reference: cuda/moe_dispatch.cu:16-45 (serial counting sort, stable in
// token-then-slot order) and the atomic count/scan/scatter of
// cuda/qgemm.cu:966-989 (whose order inside an expert is nondeterministic).
// Here the order is the reference's stable one and the work is parallel:
//   1. LDS histogram (atomics on counts only: order-free),
//   2. a one-wave prefix scan over experts,
//   3. rows in chunks of NT in input order; inside a wave, equal expert ids
//      are matched with one ballot per id bit (rank = lanes below with the
//      same id); across the waves of a chunk, per-wave counts in LDS give
//      each row the number of equal ids in earlier waves. The result is a
//      pure function of topk_ids.
#pragma once
#include "common.hpp"
#include "kernels.hpp"

namespace glmmoe {

constexpr int kDispMaxE = 512;

// Exclusive prefix of vals[0..count) (count <= 576: 512 experts and the
// shared one) into pre[0..count], pre[count] = total, by wave 0 alone: each
// lane sums 9 consecutive entries, then a wave scan of the lane sums. Callers
// synchronize before and after.
__device__ inline void wave0_exclusive_scan(const int* vals, int count, int* pre) {
    constexpr int kPer = 9;
    const int lane = threadIdx.x & 63;
    if (threadIdx.x >= 64) return;
    int local[kPer];
    int sum = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = lane * kPer + j;
        local[j] = i < count ? vals[i] : 0;
        sum += local[j];
    }
    int incl = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(incl, off);
        if (lane >= off) incl += t;
    }
    int run = incl - sum;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = lane * kPer + j;
        if (i < count) pre[i] = run;
        run += local[j];
    }
    if (lane == 63) pre[count] = incl;
}

// The whole dispatch, by one workgroup of NT threads (all of them call it).
// LDS ints dispatch_block<NT> uses.
template <int NT>
__host__ __device__ constexpr int dispatch_lds_ints() {
    return 4 * (kDispMaxE + 2) + (NT / 64) * kDispMaxE;
}

// COH: read ids with device-coherent loads (ids written by other workgroups
// of the same launch). lds: dispatch_lds_ints<NT>() ints of LDS.
// Multi-workgroup form: this workgroup permutes ids [i0, i1) (chunk blk of
// nblk); bcounts [nblk][E] holds every chunk's expert histogram, from which
// the expert bases and this chunk's start inside each expert follow; chunk 0
// also writes the offsets, the shared rows and the tile list. With
// bcounts == nullptr the workgroup does the whole dispatch alone.
template <int NT, bool COH = false>
__device__ void dispatch_block(const int* __restrict__ ids, int n, int topk, int E,
                               const DispOut& d, int* lds, int i0 = 0, int i1 = -1,
                               const int* __restrict__ bcounts = nullptr, int nblk = 1,
                               int blk = 0) {
    auto id_at = [&](int i) { return COH ? ld_dev(ids + i) : ids[i]; };
    int* cnt = lds;
    int* cursor = cnt + (kDispMaxE + 2);
    int* pre = cursor + (kDispMaxE + 2);
    int* ntl = pre + (kDispMaxE + 2);
    int (*wc)[kDispMaxE] = reinterpret_cast<int (*)[kDispMaxE]>(ntl + (kDispMaxE + 2));
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int total = n * topk;
    int nbits = 0;
    while ((1 << nbits) < E) ++nbits;

    if (i1 < 0) i1 = total;
    // One workgroup doing the whole dispatch: the ids of its first kIdRegs
    // passes are loaded once, up front (their latency under the clearing
    // below), and serve both the histogram and the permutation.
    constexpr int kIdRegs = 4;
    const bool cached = !bcounts;
    int idr[kIdRegs];
#pragma unroll
    for (int j = 0; j < kIdRegs; ++j) {
        const int i = tid + j * NT;
        idr[j] = cached && i < total ? id_at(i) : -1;
    }
    if (blk == 0 && d.zero)
        for (int i = tid; i < d.nzero; i += NT) d.zero[i] = 0u;
    for (int e = tid; e <= kDispMaxE; e += NT) cnt[e] = 0;
    for (int i = tid; i < (NT / 64) * kDispMaxE; i += NT) (&wc[0][0])[i] = 0;
    __syncthreads();
    if (bcounts) {
        // cnt = the experts' totals; ntl (scratch here) = ids of expert e in
        // the chunks before this one.
        for (int e = tid; e < E; e += NT) {
            int before = 0, all = 0;
            for (int b = 0; b < nblk; ++b) {
                const int c = bcounts[(size_t)b * E + e];
                before += b < blk ? c : 0;
                all += c;
            }
            cnt[e] = all;
            ntl[e] = before;
        }
    } else {
#pragma unroll
        for (int j = 0; j < kIdRegs; ++j)
            if (idr[j] >= 0 && idr[j] < E) atomicAdd(&cnt[idr[j]], 1);
        for (int i = tid + kIdRegs * NT; i < total; i += NT) {
            const int e = id_at(i);
            if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
        }
    }
    __syncthreads();

    // Exclusive prefix over experts.
    wave0_exclusive_scan(cnt, E, pre);
    __syncthreads();
    const bool lead = blk == 0;
    for (int e = tid; e <= E; e += NT) {
        if (lead) d.offsets[e] = pre[e];
        if (e < E) cursor[e] = pre[e] + (bcounts ? ntl[e] : 0);
    }
    if (lead && (d.mode & 1) && tid == 0) d.offsets[E + 1] = total + (d.with_shared ? n : 0);
    __syncthreads();

    // Stable permute.
    for (int base = i0, pass = 0; base < i1; base += NT, ++pass) {
        const int i = base + tid;
        int e;
        if (cached && pass < kIdRegs)
            e = pass == 0 ? idr[0] : pass == 1 ? idr[1] : pass == 2 ? idr[2] : idr[3];
        else
            e = i < i1 ? id_at(i) : -1;
        const bool valid = e >= 0 && e < E;
        uint64_t m = __ballot(valid);
        for (int b = 0; b < nbits; ++b) {
            const bool bit = valid && ((e >> b) & 1);
            const uint64_t bal = __ballot(bit);
            m &= bit ? bal : ~bal;
        }
        const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
        const int rank = __popcll(m & below);
        const bool leader = valid && rank == 0;
        if (leader) wc[wv][e] = __popcll(m);
        __syncthreads();
        if (valid) {
            int earlier = 0;
            for (int w = 0; w < wv; ++w) earlier += wc[w][e];
            const int pos = cursor[e] + earlier + rank;
            d.sorted_tok[pos] = i / topk;
            d.sorted_slot[pos] = i % topk;
            if (d.mode & 1) d.inv[i] = pos;
        }
        __syncthreads();
        if (leader) {
            atomicAdd(&cursor[e], wc[wv][e]);
            wc[wv][e] = 0;
        }
        __syncthreads();
    }

    if (!(d.mode & 1) || !lead) return;
    // The tile list below takes each expert's first row as cursor - count,
    // i.e. it needs the cursors at the experts' ends. One workgroup doing the
    // whole dispatch leaves them there; a chunk's cursors stop at its own ids.
    if (bcounts) {
        for (int e = tid; e < E; e += NT) cursor[e] = pre[e] + cnt[e];
        __syncthreads();
    }

    // Shared-expert rows: one per token, after all routed rows.
    if (d.with_shared)
        for (int t = tid; t < n; t += NT) {
            d.sorted_tok[total + t] = t;
            d.sorted_slot[total + t] = -1;
        }

    // Tile list: expert e (e == E is the shared expert) contributes
    // ceil(count / d.tile_rows) tiles of at most d.tile_rows consecutive rows,
    // {e, first row, rows, j | m << 16}: tile j of the expert's m consecutive
    // (full-class) tiles; the half and quarter tiles carry 0 there.
    // With d.half_rows = HR > 0 an expert's last partial tile is classed by
    // its rows: at most HR / 2 ("quarter"), at most HR ("half"), or more
    // (full). The list holds the full tiles first (ntiles[1] of them), then
    // the half tiles (up to ntiles[2]), then the quarter tiles, each class in
    // expert order; ntiles[0] counts all. With half_rows == 0 every tile is
    // full (ntiles[1] = ntiles[2] = ntiles[0]); below 0 only ntiles[0] is
    // written.
    static_assert(NT / 64 >= 8, "four scan arrays in the per-wave count area");
    const int nexp = E + (d.with_shared ? 1 : 0);
    const int T = d.tile_rows, HR = d.half_rows;
    // nexp <= 513 counts and nexp + 1 prefixes: each may run into the next row.
    int* nhalf = &wc[0][0];
    int* prehalf = &wc[2][0];
    int* nq = &wc[4][0];
    int* preq = &wc[6][0];
    for (int e = tid; e < nexp; e += NT) {
        const int ce = e < E ? cnt[e] : n;
        const int full = ce / T, rem = ce - full * T;
        const bool quarter = HR > 0 && rem > 0 && rem <= HR / 2;
        const bool half = HR > 0 && rem > HR / 2 && rem <= HR;
        ntl[e] = full + (rem > 0 && !half && !quarter ? 1 : 0);
        nhalf[e] = half ? 1 : 0;
        nq[e] = quarter ? 1 : 0;
    }
    __syncthreads();
    wave0_exclusive_scan(ntl, nexp, pre);
    __syncthreads();
    if (HR > 0) {
        wave0_exclusive_scan(nhalf, nexp, prehalf);
        __syncthreads();
        wave0_exclusive_scan(nq, nexp, preq);
    }
    __syncthreads();
    for (int e = tid; e < nexp; e += NT) {
        const int ce = e < E ? cnt[e] : n;
        const int row0 = e < E ? cursor[e] - ce : total;  // cursor ended at offset + count
        const int tbase = pre[e];
        for (int j = 0; j < ntl[e]; ++j)
            d.tiles[tbase + j] = make_int4(e, row0 + j * T, min(T, ce - j * T), j | (ntl[e] << 16));
        const int full = ce / T;
        if (nhalf[e]) d.tiles[pre[nexp] + prehalf[e]] = make_int4(e, row0 + full * T, ce - full * T, 0);
        if (nq[e])
            d.tiles[pre[nexp] + prehalf[nexp] + preq[e]] = make_int4(e, row0 + full * T, ce - full * T, 0);
    }
    if (tid == 0) {
        const int nfull = pre[nexp];
        const int nh = HR > 0 ? prehalf[nexp] : 0, nqq = HR > 0 ? preq[nexp] : 0;
        d.ntiles[0] = nfull + nh + nqq;
        if (HR >= 0) {   // HR < 0: the caller's ntiles holds one int
            d.ntiles[1] = nfull;
            d.ntiles[2] = nfull + nh;
        }
    }
}

// Small-batch dispatch: the outputs dispatch_block gives (mode 1,
// half_rows 0) for total = n * topk <= 64 ids of n <= tile_rows tokens, so
// that every expert, and the shared expert, has a single tile. One wave holds
// the ids (lane j: id j) and finds equal ids with one ballot per id bit;
// a packed LDS histogram (count + 65536 per distinct expert) scanned once
// gives every expert both the number of valid ids below it (its offset) and
// the number of distinct experts below it (its tile's index). Id j lands at
// offset(e_j) + #{k < j : e_k == e_j}: the stable token-then-slot order.
// ids: in LDS, visible to every thread; hist: E + 2 ints and pre: E + 2
// ints of LDS scratch. Every output goes to ltiles / lnt / ltok (LDS) and,
// when lead, to every pointer of gd. All NT threads call it.
constexpr int kSmallDispIds = 64;

template <int NT>
__device__ void dispatch_small(const int* ids, int n, int topk, int E, int with_shared,
                               int4* ltiles, int* lnt, int* ltok, const DispOut& gd, bool lead,
                               int* hist, int* pre) {
    static_assert(NT >= kSmallDispIds, "one wave holds every id");
    const int tid = threadIdx.x, lane = tid & 63;
    const int total = n * topk;
    for (int e = tid; e <= E; e += NT) hist[e] = 0;
    int e = -1, before = 0;
    bool valid = false;
    if (tid < 64) {
        e = lane < total ? ids[lane] : -1;
        valid = e >= 0 && e < E;
        int nbits = 0;
        while ((1 << nbits) < E) ++nbits;
        uint64_t m = __ballot(valid);
        for (int b = 0; b < nbits; ++b) {
            const bool bit = valid && ((e >> b) & 1);
            const uint64_t bal = __ballot(bit);
            m &= bit ? bal : ~bal;
        }
        const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        before = __popcll(m & below);
    }
    __syncthreads();
    if (valid) atomicAdd(&hist[e], before == 0 ? 0x10001 : 1);
    __syncthreads();
    wave0_exclusive_scan(hist, E + 1, pre);
    __syncthreads();
    if (valid) {
        const int pos = (pre[e] & 0xffff) + before;
        ltok[pos] = tid / topk;
        if (lead) {
            gd.sorted_tok[pos] = tid / topk;
            gd.sorted_slot[pos] = tid % topk;
            gd.inv[tid] = pos;
        }
    }
    if (with_shared && tid < n) {
        ltok[total + tid] = tid;
        if (lead) {
            gd.sorted_tok[total + tid] = tid;
            gd.sorted_slot[total + tid] = -1;
        }
    }
    for (int x = tid; x <= E; x += NT) {
        const int p = pre[x], below = p & 0xffff, dbelow = p >> 16;
        const int cnt = x < E ? hist[x] & 0xffff : 0;
        if (lead) gd.offsets[x] = below;
        if (cnt > 0) {
            const int4 t = make_int4(x, below, cnt, 1 << 16);
            ltiles[dbelow] = t;
            if (lead) gd.tiles[dbelow] = t;
        }
        if (x == E) {
            if (with_shared) {
                const int4 t = make_int4(E, total, n, 1 << 16);
                ltiles[dbelow] = t;
                if (lead) gd.tiles[dbelow] = t;
            }
            const int nt = dbelow + (with_shared ? 1 : 0);
            lnt[0] = lnt[1] = lnt[2] = nt;
            if (lead) {
                gd.offsets[E + 1] = total + (with_shared ? n : 0);
                gd.ntiles[0] = gd.ntiles[1] = gd.ntiles[2] = nt;
            }
        }
    }
}

}  // namespace glmmoe
