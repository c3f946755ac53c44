// Router: bf16 router-logit GEMM in a fixed reduction order, and the
// wave64 sigmoid + bias top-k selection.
//
// Reference: src/model_gpu.cpp:1448-1450 (gemm_linear on the router, then
// moe_router), cuda/moe_router.cu:17-79, src/model_glm52.cpp:1105-1129.
#include "common.hpp"
#include "dispatch.hpp"
#include "kernels.hpp"
#include "topk.hpp"

namespace glmmoe {

// ---------------------------------------------------------------------------
// Router logits in the fixed order the CPU oracle restates (chunked
// linear_forward): K is cut into chunks of 128; each (token, expert, chunk)
// partial is accumulated from zero in ascending K; a logit is the ascending
// sum of its chunk partials. bf16 products are exact in fp32, so
// fma(x, w, s) == s + x*w and both kernels below give logits bit-identical
// to the oracle's.
// ---------------------------------------------------------------------------
// Small batches, two passes.
// Pass 1: one single-wave workgroup per (64-expert block, 128-K chunk,
// 8-token group); lane = expert, keeping one running sum per token. Decode
// batches are latency-bound, so all loads are issued up front and coalesced:
// the 64 x 256-byte weight chunk rows (4 rows per load instruction) and the
// tokens' 8 x 256 activation bytes go through registers into LDS (weight rows
// padded to 272 B so the per-lane row reads hit distinct banks); then each
// weight value read feeds 8 FMAs, one per token, with the activations read
// as wave-uniform LDS broadcasts. Partials go to part [n, nchunks, E].
// Pass 2: one thread per (token, expert) loads its chunk partials (all in
// flight together) and adds them in ascending chunk order.
constexpr int kRouterTG = 8;    // tokens per wave
constexpr int kRouterKC = 128;  // K chunk
constexpr int kRouterMaxChunks = 64;
constexpr int kRouterRow = kRouterKC / 2 + 4;   // LDS dwords per weight row (+16 B pad)

__global__ __launch_bounds__(64) void router_partials_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wr, int n, int H, int E,
    float* __restrict__ part, float* __restrict__ xsum) {
    __shared__ __align__(16) uint32_t wl[64 * kRouterRow];
    __shared__ __align__(16) uint4 xs[kRouterTG][kRouterKC / 8];
    const int nchunks = (H + kRouterKC - 1) / kRouterKC;
    const int eblocks = (E + 63) / 64;
    const int lane = threadIdx.x;
    long b = blockIdx.x;
    const int c = (int)(b % nchunks); b /= nchunks;
    const int eb = (int)(b % eblocks); b /= eblocks;
    const int t0 = (int)b * kRouterTG;
    const int nt = min(kRouterTG, n - t0);
    const int k0 = c * kRouterKC;
    const int klen = min(kRouterKC, H - k0);   // multiple of 8
    const int oct = lane & 15;
    // Branch-free loads: octets past the chunk end, experts past E and tokens
    // past n re-read valid data that is never used.
    const int octc = oct * 8 < klen ? oct : 0;
    uint4 wv[16], xv[2];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int row = j * 4 + (lane >> 4);
        const int e = min(eb * 64 + row, E - 1);
        wv[j] = reinterpret_cast<const uint4*>(wr + (size_t)e * H + k0)[octc];
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int t = (lane >> 4) + 4 * j;
        xv[j] = reinterpret_cast<const uint4*>(x + (size_t)(t0 + min(t, nt - 1)) * H + k0)[octc];
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int row = j * 4 + (lane >> 4);
        *reinterpret_cast<uint4*>(&wl[row * kRouterRow + oct * 4]) = wv[j];
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) xs[(lane >> 4) + 4 * j][oct] = xv[j];
    __syncthreads();

    // Group sums of the staged activations (xsum [n, H/128]), written by the
    // first expert block: ascending K, low half then high half of each dword
    // (the order of xsum_kernel).
    if (xsum && eb == 0 && lane < nt && klen == kRouterKC) {
        float xsv = 0.0f;
        for (int j = 0; j < kRouterKC / 8; ++j) {
            const uint4 v = xs[lane][j];
            const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) { xsv += bf16_to_f32(d[q] & 0xffffu); xsv += bf16_to_f32(d[q] >> 16); }
        }
        xsum[(size_t)(t0 + lane) * nchunks + c] = xsv;
    }

    float s[kRouterTG];
#pragma unroll
    for (int t = 0; t < kRouterTG; ++t) s[t] = 0.0f;
    for (int i8 = 0; i8 < klen / 8; ++i8) {
        const uint4 w4 = *reinterpret_cast<const uint4*>(&wl[lane * kRouterRow + i8 * 4]);
        const uint32_t wd[4] = {w4.x, w4.y, w4.z, w4.w};
        float wf[8];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            wf[2 * d] = bf16_to_f32(wd[d] & 0xffffu);
            wf[2 * d + 1] = __uint_as_float(wd[d] & 0xffff0000u);
        }
#pragma unroll
        for (int t = 0; t < kRouterTG; ++t) {
            if (t < nt) {
                const uint4 x4 = xs[t][i8];
                const uint32_t xd[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    s[t] = __builtin_fmaf(bf16_to_f32(xd[d] & 0xffffu), wf[2 * d], s[t]);
                    s[t] = __builtin_fmaf(__uint_as_float(xd[d] & 0xffff0000u), wf[2 * d + 1], s[t]);
                }
            }
        }
    }
    const int e = eb * 64 + lane;
    if (e < E) {
#pragma unroll
        for (int t = 0; t < kRouterTG; ++t)
            if (t < nt) part[((size_t)(t0 + t) * nchunks + c) * E + e] = s[t];
    }
}

__global__ __launch_bounds__(256) void router_fold_kernel(const float* __restrict__ part, int n,
                                                          int nchunks, int E,
                                                          float* __restrict__ logits) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)n * E) return;
    const long t = i / E;
    const int e = (int)(i % E);
    const float* p = part + (size_t)t * nchunks * E + e;
    float v[kRouterMaxChunks];
#pragma unroll
    for (int c = 0; c < kRouterMaxChunks; ++c) v[c] = c < nchunks ? p[(size_t)c * E] : 0.0f;
    float total = 0.0f;
#pragma unroll
    for (int c = 0; c < kRouterMaxChunks; ++c)
        if (c < nchunks) total = total + v[c];
    logits[i] = total;
}

// Large batches: a VALU GEMM tiled through LDS. Workgroup = 128 threads, tile
// 32 tokens x 128 experts; thread (tt, ee) owns 8 tokens x 4 experts. K runs
// in steps of 32: the step's x [32 x 32] and w [128 x 32] are unpacked to
// fp32 once and stored k-major in LDS (double-buffered; the next step's
// global loads are in flight during the current step's FMAs), so each k costs
// a thread 3 LDS reads (x broadcast across the 32 threads of a token group)
// for 32 FMAs. Every 4 steps (one 128-K chunk) the running chunk partials are
// added into the totals in ascending chunk order and restarted from zero.
constexpr int kTiledTok = 32;
constexpr int kTiledExp = 128;
constexpr int kTiledK = 32;
constexpr int kTiledThreads = 128;
constexpr int kTiledMinTokens = 256;   // below: the small-batch kernel

__global__ __launch_bounds__(kTiledThreads) void router_logits_tiled_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wr, int n, int H, int E,
    float* __restrict__ logits) {
    __shared__ __align__(16) float xl[2][kTiledK][kTiledTok];   // [buffer][k][token]
    __shared__ __align__(16) float wl[2][kTiledK][kTiledExp];
    const int eblocks = (E + kTiledExp - 1) / kTiledExp;
    const int eb = (int)(blockIdx.x % eblocks);
    const int t0 = (int)(blockIdx.x / eblocks) * kTiledTok;
    const int e0 = eb * kTiledExp;
    const int tid = threadIdx.x;
    const int tt = tid >> 5, ee = tid & 31;     // 4 token groups x 32 expert quads
    // Staging roles: x -- token tid / 4, k-octet tid % 4; w -- expert tid, all 32 k.
    const uint4* xsrc = reinterpret_cast<const uint4*>(x + (size_t)min(t0 + (tid >> 2), n - 1) * H) + (tid & 3);
    const uint4* wsrc = reinterpret_cast<const uint4*>(wr + (size_t)min(e0 + tid, E - 1) * H);
    const int nsteps = H / kTiledK;

    uint4 xr, wrg[4];
    auto load = [&](int st) {
        xr = xsrc[st * 4];
#pragma unroll
        for (int j = 0; j < 4; ++j) wrg[j] = wsrc[st * 4 + j];
    };
    auto store = [&](int buf) {
        const uint32_t xd[4] = {xr.x, xr.y, xr.z, xr.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const int k = (tid & 3) * 8 + 2 * d;
            xl[buf][k][tid >> 2] = bf16_to_f32(xd[d] & 0xffffu);
            xl[buf][k + 1][tid >> 2] = __uint_as_float(xd[d] & 0xffff0000u);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t wd[4] = {wrg[j].x, wrg[j].y, wrg[j].z, wrg[j].w};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const int k = j * 8 + 2 * d;
                wl[buf][k][tid] = bf16_to_f32(wd[d] & 0xffffu);
                wl[buf][k + 1][tid] = __uint_as_float(wd[d] & 0xffff0000u);
            }
        }
    };

    float part[8][4], tot[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) { part[i][j] = 0.0f; tot[i][j] = 0.0f; }

    load(0);
    store(0);
    __syncthreads();
    for (int st = 0; st < nsteps; ++st) {
        const int buf = st & 1;
        if (st + 1 < nsteps) load(st + 1);
#pragma unroll 8
        for (int k = 0; k < kTiledK; ++k) {
            const float4 xa = *reinterpret_cast<const float4*>(&xl[buf][k][tt * 8]);
            const float4 xb = *reinterpret_cast<const float4*>(&xl[buf][k][tt * 8 + 4]);
            const float4 wv = *reinterpret_cast<const float4*>(&wl[buf][k][ee * 4]);
            const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            const float wf[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) part[i][j] = __builtin_fmaf(xv[i], wf[j], part[i][j]);
        }
        if ((st & 3) == 3 || st + 1 == nsteps) {   // end of a 128-K chunk
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) { tot[i][j] = tot[i][j] + part[i][j]; part[i][j] = 0.0f; }
        }
        if (st + 1 < nsteps) store(buf ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int t = t0 + tt * 8 + i;
        if (t >= n) continue;
        const int e = e0 + ee * 4;
        if (e + 3 < E && (E & 3) == 0) {
            *reinterpret_cast<float4*>(logits + (size_t)t * E + e) =
                make_float4(tot[i][0], tot[i][1], tot[i][2], tot[i][3]);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (e + j < E) logits[(size_t)t * E + e + j] = tot[i][j];
        }
    }
}

// Activation group sums alone (for callers that bring their own routing).
__global__ __launch_bounds__(256) void xsum_kernel(const uint16_t* __restrict__ x, int n,
                                                   int H, float* __restrict__ xsum) {
    const int nchunks = H / kRouterKC;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)n * nchunks) return;
    const int t = (int)(i / nchunks), c = (int)(i % nchunks);
    const uint4* p = reinterpret_cast<const uint4*>(x + (size_t)t * H + c * kRouterKC);
    float s = 0.0f;
    for (int j = 0; j < kRouterKC / 8; ++j) {
        const uint4 v = p[j];
        const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) { s += bf16_to_f32(d[q] & 0xffffu); s += bf16_to_f32(d[q] >> 16); }
    }
    xsum[i] = s;
}


// Dispatch on the experts per lane (E <= 64 * NJ). pcode / pscore: the
// token's order codes and scores when the caller computed them (else null).
template <bool COH = false>
__device__ __forceinline__ void topk_wave(const float* __restrict__ lt,
                                          const float* __restrict__ e_bias, int E, int topk,
                                          int norm_topk, float routed_scale,
                                          int* __restrict__ ids_out, float* __restrict__ w_out,
                                          uint32_t* scratch, const uint32_t* pcode = nullptr,
                                          const float* pscore = nullptr) {
#define GLMMOE_TOPK_ARGS lt, e_bias, E, topk, norm_topk, routed_scale, ids_out, w_out, scratch, pcode, pscore
    if (E <= 64) topk_wave_nj<COH, 1>(GLMMOE_TOPK_ARGS);
    else if (E <= 128) topk_wave_nj<COH, 2>(GLMMOE_TOPK_ARGS);
    else if (E <= 256) topk_wave_nj<COH, 4>(GLMMOE_TOPK_ARGS);
    else topk_wave_nj<COH, 8>(GLMMOE_TOPK_ARGS);
#undef GLMMOE_TOPK_ARGS
}

__global__ __launch_bounds__(256) void router_topk_kernel(
    const float* __restrict__ logits, const float* __restrict__ e_bias, int n, int E, int topk,
    int norm_topk, float routed_scale, int* __restrict__ topk_ids, float* __restrict__ topk_w) {
    __shared__ uint32_t scratch[4][kTopkScratch];
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n) return;   // whole wave
    topk_wave(logits + (size_t)t * E, e_bias, E, topk, norm_topk, routed_scale,
              topk_ids + (size_t)t * topk, topk_w + (size_t)t * topk, scratch[threadIdx.x >> 6]);
}

// ---------------------------------------------------------------------------
// Large batches inside the layer: routing without the fixed-order GEMM over
// every (token, expert) pair. The ids and weights are still exactly those of
// the fixed-order logits:
//   1. router_mfma_kernel: approximate logits L~ = x . w on bf16 MFMA, and
//      S = |x| . |w| (the same MFMA on sign-cleared operands). bf16 products
//      are exact in fp32, so both the fixed-order sum L and L~ are sums of the
//      same exact terms and |L~ - L| is below a small multiple of u * K * S
//      (u = 2^-24) for any fp32 summation order; eps = 2^-11 * S covers it
//      with a wide margin (2^-11 / (2 * 2^-24 * 6144) = 0.67 x the worst case
//      of two K-term sequential sums, and about 14 x the worst case of this
//      build's orders).
//   2. router_refine_kernel, one wave per token: lower/upper bounds of each
//      expert's choose value from L~ -+ eps (choose = sigmoid(logit) + bias is
//      monotone in the logit; 1e-6 absorbs sigmoid rounding); T = the k-th
//      largest lower bound. An expert whose upper bound is below T is below
//      at least k others for sure and cannot be selected. Every other expert
//      (the candidates, k plus the near ties) gets its exact fixed-order
//      logit; the rest get -inf (choose = bias < T). The wave also writes the
//      activation group sums xsum.
//   3. router_topk_kernel on those logits: the selection and weights only
//      ever read candidates' logits, so they equal the oracle's bit for bit.
// ---------------------------------------------------------------------------
constexpr int kMfmaTok = 64;   // tokens per workgroup
constexpr int kMfmaExp = 64;   // experts per workgroup
constexpr int kMfmaK = 64;     // K per LDS stage
constexpr int kMfmaD = 4;      // stages in flight + 1

// Row r of a [64 x 64] bf16 stage tile: 128 B at 128 r; 16-byte chunk c at
// slot c ^ ((r >> 1) & 7), so the 16 rows of an MFMA fragment pass read
// distinct bank groups.
__device__ __forceinline__ uint32_t mfma_tile_off(int r, int c) {
    return (uint32_t)(r * 128 + ((c ^ ((r >> 1) & 7)) << 4));
}

// Stages (64 K of 64 token rows and 64 expert rows, 16 KiB) stream into a
// kMfmaD-slot LDS ring by LDS-DMA: 4 DMAs per wave per stage, each 8 whole
// 128-B rows (lane l: row l / 8, slot l % 8 holding chunk (l % 8) ^ swz(row)).
// K split z of nsplit (blockIdx.z) covers stages [z nk / nsplit, (z + 1) nk
// / nsplit) and writes its partial L~ to lt (z = 0) or lp + (z - 1) n E, its
// partial S to sb + z n E.
__global__ __launch_bounds__(256) void router_mfma_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ wr, int n,
                                                          int H, int E, float* __restrict__ lt,
                                                          float* __restrict__ sb, float* __restrict__ lp,
                                                          int nsplit) {
    extern __shared__ __align__(16) char tl[];   // [kMfmaD][x | w][64 rows x 128 B]
    constexpr int kStage = 2 * kMfmaTok * 128;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int e0 = blockIdx.x * kMfmaExp, t0 = blockIdx.y * kMfmaTok;
    const int tb = wave & 1, eb = wave >> 1;
    // DMA j (0..3) of this wave: operand j / 2 (x, w), rows 8 (2 wave + j % 2) + lane / 8.
    const uint16_t* src[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = 8 * (2 * wave + (j & 1)) + (lane >> 3);
        const int c = (lane & 7) ^ ((row >> 1) & 7);
        const uint16_t* rp = (j >> 1) == 0 ? x + (size_t)min(t0 + row, n - 1) * H
                                           : wr + (size_t)min(e0 + row, E - 1) * H;
        src[j] = rp + c * 8;
    }
    auto issue = [&](int ks) {
        char* st = tl + (ks % kMfmaD) * kStage;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            dma16(src[j] + (size_t)ks * kMfmaK,
                  st + (j >> 1) * (kMfmaTok * 128) + (2 * wave + (j & 1)) * 1024);
    };
    f32x16 accl = {}, accs = {};
    const int ar = tb * 32 + (lane & 31), br = eb * 32 + (lane & 31), hh = lane >> 5;
    const int nkt = H / kMfmaK, z = blockIdx.z;
    const int k0 = (int)((long)nkt * z / nsplit), nk = (int)((long)nkt * (z + 1) / nsplit);
    for (int j = 0; j < kMfmaD - 1; ++j)
        if (k0 + j < nk) issue(k0 + j);
    for (int ks = k0; ks < nk; ++ks) {
        if (ks + kMfmaD - 2 < nk) wait_vmcnt<4 * (kMfmaD - 2)>();
        else wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();   // stage ks visible; stage ks - 1 free
        if (ks + kMfmaD - 1 < nk) issue(ks + kMfmaD - 1);
        const uint32_t xa = lds_addr(tl + (ks % kMfmaD) * kStage);
        const uint32_t wa = xa + kMfmaTok * 128;
        u32x4 av[4], bv[4];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            const int c = 2 * s4 + hh;
            asm volatile("ds_read_b128 %0, %2\n ds_read_b128 %1, %3"
                         : "=&v"(av[s4]), "=&v"(bv[s4])
                         : "v"(xa + mfma_tile_off(ar, c)), "v"(wa + mfma_tile_off(br, c)));
        }
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(av[0]), "+v"(av[1]), "+v"(av[2]), "+v"(av[3]), "+v"(bv[0]),
                       "+v"(bv[1]), "+v"(bv[2]), "+v"(bv[3]));
        const u32x4 m = {0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu};
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            accl = mfma32x32x16(as_bf16x8(av[s4]), as_bf16x8(bv[s4]), accl);
            accs = mfma32x32x16(as_bf16x8(av[s4] & m), as_bf16x8(bv[s4] & m), accs);
        }
    }
    // D: lane -> expert column br, rows (tokens) 8 (i / 4) + 4 hh + i % 4 of the block.
    const int e = e0 + br;
    float* lo = z == 0 ? lt : lp + (size_t)(z - 1) * n * E;
    float* so = sb + (size_t)z * n * E;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int t = t0 + tb * 32 + 8 * (i >> 2) + 4 * hh + (i & 3);
        if (t < n && e < E) {
            lo[(size_t)t * E + e] = accl[i];
            so[(size_t)t * E + e] = accs[i];
        }
    }
}

__device__ __forceinline__ float code_to_float(uint32_t c) {
    return __uint_as_float((c & 0x80000000u) ? (c & 0x7fffffffu) : ~c);
}

constexpr int kRefineWaves = 2;   // tokens (waves) per workgroup with one wave per token
// Below this many tokens each token gets kRefineSplit waves: the token waves
// then do not fill the SIMDs, and the kernel takes one token's serial chain
// of candidate passes; the waves split the candidates (every wave computes
// the same bounds and candidate list).
constexpr int kRefineSplitMax = 1024;
constexpr int kRefineSplit = 4;

// TW: waves per token (1: kRefineWaves tokens per workgroup; else one token
// per workgroup of TW waves).
template <int NJ, int TW>   // keys per lane: E <= 64 * NJ
__global__ __launch_bounds__(TW == 1 ? kRefineWaves * 64 : TW * 64) void router_refine_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wr,
    const float* __restrict__ e_bias, const float* __restrict__ sb, int n, int H, int E, int topk,
    float* __restrict__ logits, float* __restrict__ xsum, int nsplit, uint16_t* __restrict__ xh,
    float* __restrict__ xrho) {
    constexpr int TPW = TW == 1 ? kRefineWaves : 1;   // tokens per workgroup
    const int lane = threadIdx.x & 63;
    const int slot = TW == 1 ? (int)(threadIdx.x >> 6) : 0;    // token slot of this wave
    const int sub = TW == 1 ? 0 : (int)(threadIdx.x >> 6);     // this wave's share of the candidates
    const int t = blockIdx.x * TPW + slot;
    if (t >= n) return;   // whole wave (TW > 1: whole workgroup)
    const int nchunks = H / kRouterKC;
    // This lane's 128-K chunk of x (lanes past the chunk count hold zeros),
    // kept in LDS for the exact sums (registers go to the weight buffers).
    __shared__ uint4 xl[TPW][kRouterKC / 8][64];
    uint4 (*xw)[64] = xl[slot];
    if (sub == 0) {
        const uint4* xp = reinterpret_cast<const uint4*>(x + (size_t)t * H + lane * kRouterKC);
#pragma unroll
        for (int j = 0; j < kRouterKC / 8; ++j) xw[j][lane] = lane < nchunks ? xp[j] : make_uint4(0, 0, 0, 0);
    }
    if constexpr (TW > 1) __syncthreads();   // wave 0 staged the token's x
    if (xh && sub == 0) {
        // The large-group gate/up kernel's input row: x in fp16 with a
        // power-of-2 scale that puts the row's largest magnitude in
        // [2^14, 2^15), and the factor undoing it (times 2^-kWPre): the rule
        // and operations of f16_rows_kernel, from the staged row.
        uint32_t amax = 0;   // bf16 magnitudes compare as integers
        if (lane < nchunks) {
#pragma unroll
            for (int j = 0; j < kRouterKC / 8; ++j) {
                const uint4 v = xw[j][lane];
                const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    amax = max(amax, d[q] & 0x7fffu);
                    amax = max(amax, (d[q] >> 16) & 0x7fffu);
                }
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) amax = max(amax, (uint32_t)__shfl_xor((int)amax, off));
        const int ex = amax >= 0x0080u ? (int)(amax >> 7) - 127 : 0;
        int kx = 14 - ex;
        kx = kx > 100 ? 100 : (kx < -100 ? -100 : kx);
        const float scale = __builtin_ldexpf(1.0f, kx);
        if (lane == 0) xrho[t] = __builtin_ldexpf(1.0f, -kx - kWPre);
        if (lane < nchunks) {
            uint4* yr = reinterpret_cast<uint4*>(xh + (size_t)t * H + lane * kRouterKC);
#pragma unroll
            for (int j = 0; j < kRouterKC / 8; ++j) {
                const uint4 v = xw[j][lane];
                const uint32_t d[4] = {v.x, v.y, v.z, v.w};
                uint32_t o[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const _Float16 lo = (_Float16)(bf16_to_f32(d[q] & 0xffffu) * scale);
                    const _Float16 hi = (_Float16)(bf16_to_f32(d[q] >> 16) * scale);
                    o[q] = (uint32_t)__builtin_bit_cast(uint16_t, lo) |
                           ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
                }
                yr[j] = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
    }
    if (xsum && sub == 0 && lane < nchunks) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < kRouterKC / 8; ++j) {
            const uint4 xv = xw[j][lane];
            const uint32_t d[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) { s += bf16_to_f32(d[q] & 0xffffu); s += bf16_to_f32(d[q] >> 16); }
        }
        xsum[(size_t)t * nchunks + lane] = s;
    }
    float* lrow = logits + (size_t)t * E;
    const float* srow = sb + (size_t)t * E;
    uint32_t lo[NJ];   // order codes of the lower bounds (0 = none / taken)
    float up[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int e = lane + 64 * j;
        lo[j] = 0u;
        up[j] = -INFINITY;
        if (e < E) {
            // The K splits' partials, added in split order (any order keeps
            // L~ a sum of the same exact products: the bound below holds).
            float l = lrow[e], sabs = srow[e];
            for (int z = 1; z < nsplit; ++z) {
                l = l + sb[(size_t)nsplit * n * E + (size_t)(z - 1) * n * E + (size_t)t * E + e];
                sabs = sabs + sb[(size_t)z * n * E + (size_t)t * E + e];
            }
            const float eps = sabs * 0x1p-11f;
            const float b = e_bias ? e_bias[e] : 0.0f;
            if (l != l || eps != eps) {
                up[j] = INFINITY;    // always a candidate; never sets the threshold
                lo[j] = 1u;
            } else {
                lo[j] = order_code(sigmoid_fixed(l - eps) + b - 1e-6f);
                up[j] = sigmoid_fixed(l + eps) + b + 1e-6f;
            }
        }
    }
    // T = k-th largest lower bound (counted with multiplicity): each round
    // takes the largest remaining code and drops all its copies, until k
    // codes are covered.
    uint32_t tcode = 0u;
    int remaining = topk;
    for (int k = 0; k < topk && remaining > 0; ++k) {
        uint32_t m = lo[0];
#pragma unroll
        for (int j = 1; j < NJ; ++j) m = lo[j] > m ? lo[j] : m;
        const uint32_t bh = wave_umax(m);
        int c = 0;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const bool hit = lo[j] == bh;
            c += __builtin_popcountll(__ballot(hit));
            lo[j] = hit ? 0u : lo[j];
        }
        tcode = bh;
        remaining -= c;
    }
    const float T = tcode > 1u ? code_to_float(tcode) : -INFINITY;
    // Candidates in ascending expert order into this wave's LDS list; the rest
    // get -inf.
    __shared__ int cl[TPW * TW][64 * NJ];
    int* list = cl[threadIdx.x >> 6];
    int ncand = 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int e = lane + 64 * j;
        const bool cand = e < E && up[j] >= T;
        if (sub == 0 && e < E && !cand) lrow[e] = -INFINITY;
        const uint64_t mask = __ballot(cand);
        const int before = __builtin_popcountll(mask & ((1ull << lane) - 1));
        if (cand) list[ncand + before] = e;
        ncand += __builtin_popcountll(mask);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): list writes done
    __builtin_amdgcn_wave_barrier();
    // Exact fixed-order logits of the candidates: lane c sums chunk c in
    // ascending K, then the chunk sums are added in ascending c. Occupancy
    // (few registers per wave) hides the weight loads.
    // Two candidates at a time: their loads in flight together and their
    // chains interleaved (each chain is still the ascending-K sum from zero).
    for (int i = 2 * sub; i < ncand; i += 2 * TW) {
        const bool two = i + 1 < ncand;
        const int ec0 = list[i], ec1 = two ? list[i + 1] : ec0;
        const uint4* wp0 = reinterpret_cast<const uint4*>(wr + (size_t)ec0 * H + lane * kRouterKC);
        const uint4* wp1 = reinterpret_cast<const uint4*>(wr + (size_t)ec1 * H + lane * kRouterKC);
        float p0 = 0.0f, p1 = 0.0f;
        if (lane < nchunks) {
            uint4 w0[kRouterKC / 8], w1[kRouterKC / 8];
#pragma unroll
            for (int q = 0; q < kRouterKC / 8; ++q) { w0[q] = wp0[q]; w1[q] = wp1[q]; }
#pragma unroll
            for (int q = 0; q < kRouterKC / 8; ++q) {
                const uint4 xv = xw[q][lane];
                const uint32_t xd[4] = {xv.x, xv.y, xv.z, xv.w};
                const uint32_t a[4] = {w0[q].x, w0[q].y, w0[q].z, w0[q].w};
                const uint32_t b[4] = {w1[q].x, w1[q].y, w1[q].z, w1[q].w};
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const float xlo = bf16_to_f32(xd[d] & 0xffffu), xhi = __uint_as_float(xd[d] & 0xffff0000u);
                    p0 = __builtin_fmaf(xlo, bf16_to_f32(a[d] & 0xffffu), p0);
                    p1 = __builtin_fmaf(xlo, bf16_to_f32(b[d] & 0xffffu), p1);
                    p0 = __builtin_fmaf(xhi, __uint_as_float(a[d] & 0xffff0000u), p0);
                    p1 = __builtin_fmaf(xhi, __uint_as_float(b[d] & 0xffff0000u), p1);
                }
            }
        }
        // ((0 + p_0) + p_1) + ... in chunk order, as a ripple across lanes:
        // each step every lane adds its own partial to its left neighbour's
        // running sum (wave shift right by one; lane 0 reads 0). After
        // nchunks - 1 steps lane nchunks - 1 holds the whole ordered sum.
        float t0 = 0.0f + p0, t1 = 0.0f + p1;
        for (int c = 1; c < nchunks; ++c) {
            t0 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t0), 0x138, 0xf, 0xf, true)) + p0;
            t1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t1), 0x138, 0xf, 0xf, true)) + p1;
        }
        if (lane == nchunks - 1) {
            lrow[ec0] = t0;
            if (two) lrow[ec1] = t1;
        }
    }
}

// ---------------------------------------------------------------------------
// Small batches inside the layer (n < kTiledMinTokens): router_small_kernel
// computes the logits and the selection's inputs (order codes, scores), then
// router_finish_kernel selects and (n <= kFinishDispMax) dispatches.
// Grid (ceil(E / epw), ceil(n / 8)) of 512 threads. The group's activations
// are staged in LDS; thread (expert eb * epw + el, chunk c, token slice ts)
// keeps the chunk's 128 router weights in registers and, for each token of
// its slice, accumulates the chunk partial from zero in ascending K (the
// fixed order of router_partials_kernel). Threads (expert, token) then add
// the chunk partials in ascending chunk order: the logit, bit-identical to
// the two-pass path. No state outlives a launch: two launches may overlap on
// different streams.
// ---------------------------------------------------------------------------
constexpr int kSmallThreads = 512;
constexpr int kSmallMaxChunks = 64;
constexpr int kFinishDispMax = 8;   // tokens up to which one workgroup selects and dispatches
// Staged activation bytes: 8 tokens x nchunks rows of 256 B, whole 1 KiB DMAs.
__host__ __device__ constexpr int small_x_bytes(int nchunks) {
    return (kRouterTG * nchunks * 256 + 1023) / 1024 * 1024;
}

// NT independent token chains over one 128-K chunk c: the ascending-K sum
// from zero of x[t] * w, for tokens tb + t, t < nt (rows past nt repeat the
// last one and are not stored). The NT activation pieces of step j + 1 are read from
// LDS while step j is computed.
template <int NT>
__device__ __forceinline__ void small_chunk_dots(const char* xl, const uint4 (&wv)[kRouterKC / 8],
                                                 int c, int nchunks, int tb, int nt, float* out) {
    uint32_t base[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int R = (tb + (t < nt ? t : nt - 1)) * nchunks + c;
        base[t] = (uint32_t)(R * 256);
    }
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    auto rd = [&](int j, uint4 (&xv)[NT]) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint32_t R15 = (base[t] >> 8) & 15;
            xv[t] = *reinterpret_cast<const uint4*>(xl + base[t] + (((uint32_t)j ^ R15) << 4));
        }
    };
    uint4 xa[NT], xb[NT];
    rd(0, xa);
#pragma unroll
    for (int j = 0; j < kRouterKC / 8; ++j) {
        uint4 (&cur)[NT] = (j & 1) ? xb : xa;
        uint4 (&nxt)[NT] = (j & 1) ? xa : xb;
        if (j + 1 < kRouterKC / 8) rd(j + 1, nxt);
        const uint32_t wd[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
        float wf[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            wf[2 * q] = bf16_to_f32(wd[q] & 0xffffu);
            wf[2 * q + 1] = __uint_as_float(wd[q] & 0xffff0000u);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint32_t xd[4] = {cur[t].x, cur[t].y, cur[t].z, cur[t].w};
                acc[t] = __builtin_fmaf(bf16_to_f32(xd[q] & 0xffffu), wf[2 * q], acc[t]);
                acc[t] = __builtin_fmaf(__uint_as_float(xd[q] & 0xffff0000u), wf[2 * q + 1], acc[t]);
            }
        // Pin each step's chains here (otherwise the reads of every step are
        // hoisted and the arithmetic sunk, holding 16 * NT pieces live).
#pragma unroll
        for (int t = 0; t < NT; ++t) asm volatile("" : "+v"(acc[t]));
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
        if (t < nt) out[tb + t] = acc[t];
}

// ((0 + p[0]) + p[stride]) + ... over count partials, in that order; the
// loads go out 8 at a time ahead of the dependent adds.
__device__ __forceinline__ float chunk_sum(const float* p, int stride, int count) {
    float total = 0.0f;
    int c = 0;
    for (; c + 8 <= count; c += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p[(c + u) * stride];
#pragma unroll
        for (int u = 0; u < 8; ++u) total = total + v[u];
    }
    for (; c < count; ++c) total = total + p[c * stride];
    return total;
}

__global__ __launch_bounds__(kSmallThreads) void router_small_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wr,
    const float* __restrict__ e_bias, int n, int H, int E, int epw, float* __restrict__ logits,
    float* __restrict__ xsum, int slices, uint32_t* __restrict__ cs, unsigned int* __restrict__ zero,
    int nzero, const float* __restrict__ xf, uint16_t* __restrict__ xb) {
    extern __shared__ __align__(16) char small_lds[];
    const int nchunks = H / kRouterKC;
    const int tid = threadIdx.x;
    const int eb = blockIdx.x, tg = blockIdx.y;
    // The expert kernels' tickets, when the selection runs inside gate/up.
    if (zero && eb == 0 && tg == 0)
        for (int i = tid; i < nzero; i += kSmallThreads) zero[i] = 0u;
    const int t0 = tg * kRouterTG, nt = min(kRouterTG, n - t0);
    // LDS: the group's activations as 256-byte rows R = t * nchunks + c
    // (token t, chunk c), 16-byte piece o of row R at slot o ^ (R & 15) (the
    // threads of consecutive chunks reading the same piece hit distinct
    // banks), staged by LDS-DMA, 1 KiB (4 rows) per wave instruction; then
    // the chunk partials part[thread][token].
    char* xl = small_lds;
    const int xrows = nt * nchunks;
    const int xdma = (xrows + 3) / 4;
    float* part = reinterpret_cast<float*>(small_lds + small_x_bytes(nchunks));
    if (!xf) {
        const int wave = tid >> 6, lane = tid & 63;
        for (int b = wave; b < xdma; b += kSmallThreads / 64) {
            int R = 4 * b + (lane >> 4);
            if (R >= xrows) R = 0;
            const int t = R / nchunks, cc = R - t * nchunks;
            const int o = (lane & 15) ^ (R & 15);
            dma16(x + (size_t)(t0 + t) * H + cc * kRouterKC + o * 8, xl + b * 1024);
        }
    } else {
        // fp32 activations: the same 16-B pieces, each from 8 fp32 values
        // rounded to bf16 (nearest even) on the way into LDS; the first
        // expert block also writes the rounded rows to xb for the expert
        // kernels, so the layer reads fp32 x once and needs no cast launch.
        const int wave = tid >> 6, lane = tid & 63;
        for (int b = wave; b < xdma; b += kSmallThreads / 64) {
            const int R = 4 * b + (lane >> 4);
            if (R >= xrows) continue;
            const int t = R / nchunks, cc = R - t * nchunks;
            const int o = (lane & 15) ^ (R & 15);
            const size_t off = (size_t)(t0 + t) * H + cc * kRouterKC + o * 8;
            const float4 lo = *reinterpret_cast<const float4*>(xf + off);
            const float4 hi = *reinterpret_cast<const float4*>(xf + off + 4);
            const uint4 v = make_uint4(f32_to_bf16(lo.x) | (f32_to_bf16(lo.y) << 16),
                                       f32_to_bf16(lo.z) | (f32_to_bf16(lo.w) << 16),
                                       f32_to_bf16(hi.x) | (f32_to_bf16(hi.y) << 16),
                                       f32_to_bf16(hi.z) | (f32_to_bf16(hi.w) << 16));
            *reinterpret_cast<uint4*>(xl + b * 1024 + lane * 16) = v;
            if (eb == 0) *reinterpret_cast<uint4*>(xb + off) = v;
        }
    }
    // Thread -> (expert el, chunk c, token slice ts): slice ts holds tokens
    // [ts * tps, ts * tps + tps) of the group.
    const int ec = epw * nchunks;
    const int pair = tid % ec, ts = tid / ec;
    const int el = pair / nchunks, c = pair - el * nchunks;
    const int e = eb * epw + el;
    const int tps = kRouterTG / slices;
    const int tb = ts * tps, tcnt = min(tps, nt - tb);
    const bool active = ts < slices && e < E && tcnt > 0;
    uint4 wv[kRouterKC / 8];
    if (active) {
        const uint4* wp = reinterpret_cast<const uint4*>(wr + (size_t)e * H + c * kRouterKC);
#pragma unroll
        for (int j = 0; j < kRouterKC / 8; ++j) wv[j] = wp[j];
    }
    wait_vmcnt<0>();
    __syncthreads();
    if (active) {
        float* out = part + pair * kRouterTG;
        if (tcnt == 1) small_chunk_dots<1>(xl, wv, c, nchunks, tb, tcnt, out);
        else if (tcnt == 2) small_chunk_dots<2>(xl, wv, c, nchunks, tb, tcnt, out);
        else if (tcnt <= 4) small_chunk_dots<4>(xl, wv, c, nchunks, tb, tcnt, out);
        else small_chunk_dots<8>(xl, wv, c, nchunks, tb, tcnt, out);
    }
    // Activation group sums (xsum [n, H/128]) from the staged rows, by the
    // first expert block: ascending K, low half then high half of each dword.
    if (xsum && eb == 0) {
        for (int i = tid; i < nt * nchunks; i += kSmallThreads) {
            const int t = i / nchunks, cc = i - t * nchunks;
            const int R = t * nchunks + cc;
            const char* row = xl + R * 256;
            float xs = 0.0f;
            for (int j = 0; j < kRouterKC / 8; ++j) {
                const uint4 v = *reinterpret_cast<const uint4*>(row + ((j ^ (R & 15)) << 4));
                const uint32_t xd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    xs += bf16_to_f32(xd[q] & 0xffffu);
                    xs += bf16_to_f32(xd[q] >> 16);
                }
            }
            xsum[(size_t)(t0 + t) * nchunks + cc] = xs;
        }
    }
    __syncthreads();
    if (tid < epw * kRouterTG) {
        const int el2 = tid / kRouterTG, t = tid % kRouterTG;
        const int e2 = eb * epw + el2;
        if (e2 < E && t < nt) {
            const float total = chunk_sum(part + el2 * nchunks * kRouterTG + t, kRouterTG, nchunks);
            st_dev(logits + (size_t)(t0 + t) * E + e2, total);
            // The selection's inputs, computed here in parallel: the score
            // and the order code of choose = score + bias.
            const float sc = sigmoid_fixed(total);
            const size_t o = (size_t)(t0 + t) * E + e2;
            st_dev(cs + o, order_code(sc + (e_bias ? e_bias[e2] : 0.0f)));
            st_dev(reinterpret_cast<float*>(cs) + (size_t)n * E + o, sc);
        }
    }
}

// The selection and, for a small batch, the dispatch after router_small_kernel:
// wave w of workgroup b selects tokens 8 b + w, 8 b + w + 8 * gridDim.x, ...
// from the order codes and scores; with do_disp the grid is one workgroup,
// which then runs the whole dispatch on the ids its waves stored.
template <int NJ>
__global__ __launch_bounds__(kSmallThreads) void router_finish_kernel(
    const float* __restrict__ logits, const float* __restrict__ e_bias, int n, int E, int topk,
    int norm_topk, float routed_scale, int* __restrict__ ids, float* __restrict__ w,
    const uint32_t* __restrict__ cs, DispOut d, int do_disp) {
    __shared__ int lds[dispatch_lds_ints<kSmallThreads>()];
    __shared__ uint32_t tscratch[kSmallThreads / 64][kTopkScratch];
    __shared__ int sids[kFinishDispMax * 8];   // the dispatch's copy of the ids
    const int wave = threadIdx.x >> 6;
    for (int t = blockIdx.x * (kSmallThreads / 64) + wave; t < n; t += gridDim.x * (kSmallThreads / 64))
        topk_wave_nj<false, NJ>(logits + (size_t)t * E, e_bias, E, topk, norm_topk, routed_scale,
                                ids + (size_t)t * topk, w + (size_t)t * topk, tscratch[wave],
                                cs + (size_t)t * E,
                                reinterpret_cast<const float*>(cs) + (size_t)n * E + (size_t)t * E,
                                do_disp ? sids + t * topk : nullptr);
    if (!do_disp) return;
    __syncthreads();
    dispatch_block<kSmallThreads>(sids, n, topk, E, d, lds);
}

// ---------------------------------------------------------------------------
// Mid-size batches (kGemvMinTokens <= n < kTiledMinTokens, selection in the
// same call): router_gemv_kernel, then router_fold_select_kernel. Together
// they replace the reference's router GEMM, top-k and dispatch launches
// (src/model_gpu.cpp:1448-1450 -> cuda/gemm.cu:62-77, cuda/moe_router.cu:17-72,
// cuda/moe_dispatch.cu:16-45) with the fixed summation order of this build.
// router_gemv_kernel: grid (nchunks, ceil(E / 64), ceil(n / (4 NT))) of 4
// waves. Workgroup (c, eb, tg) takes the 128-K chunk c and the 64 experts of
// block eb: their 256-B weight rows are staged once by LDS-DMA (whole cache
// lines per instruction, 16-B pieces XOR-swizzled by row) and lane l keeps
// row 64 eb + l in registers. Wave w takes tokens 4 NT tg + NT w .. + NT,
// whose chunk activations the workgroup stages into LDS as fp32 (converted
// once); the FMAs read them as LDS broadcasts, one step (8 K) ahead, and each
// weight is converted once for the NT tokens: about one vector instruction
// per product. Each lane writes the ascending-K chain from zero of every
// token (the fixed chunk order of router_partials_kernel) to part[c][t][e];
// the first expert block's lanes t < NT also write the chunk's activation
// sums xsum[t][c] (ascending K).
// router_fold_select_kernel: one workgroup per token adds the chunk partials
// in chunk order ((0 + p0) + p1) + ..., writes the logits, and one wave
// selects: the logit of every expert bit-identical to the other paths.
// ---------------------------------------------------------------------------
constexpr int kGemvMinTokens = 9;
constexpr int kGemvWaves = 4;   // token groups (waves) per workgroup

template <int NT>
__global__ __launch_bounds__(64 * kGemvWaves) void router_gemv_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wr, int n, int H, int E,
    float* __restrict__ part, float* __restrict__ xsum, unsigned int* __restrict__ fold_ticket,
    const float* __restrict__ xf, uint16_t* __restrict__ xb) {
    constexpr int TPB = kGemvWaves * NT;   // tokens of the workgroup
    constexpr int NTH = 64 * kGemvWaves;
    // LDS: the tokens' chunk activations as fp32, xl[t][k], first (their
    // reads then fit the instruction's offset field), then the weight rows.
    __shared__ __align__(16) char glds[TPB * kRouterKC * 4 + 64 * 256];
    float (*xl)[kRouterKC] = reinterpret_cast<float (*)[kRouterKC]>(glds);
    char* wl = glds + TPB * kRouterKC * 4;
    const int nchunks = H / kRouterKC;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c = blockIdx.x;
    const int e = blockIdx.y * 64 + lane;
    const int tb = blockIdx.z * TPB, nb = min(TPB, n - tb);
    // The fold kernel's ticket (nothing in this launch reads it).
    if (fold_ticket && tid == 0 && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0)
        reset_dev(fold_ticket);
    // Weight rows of the 64 experts: 16 DMAs of 4 rows, 4 per wave; piece o
    // of row R at slot o ^ (R & 15), so the lanes reading their own rows hit
    // distinct banks.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int b = wave * 4 + i;
        const int R = 4 * b + (lane >> 4);
        const int er = min((int)blockIdx.y * 64 + R, E - 1);
        const int o = (lane & 15) ^ (R & 15);
        dma16(wr + (size_t)er * H + c * kRouterKC + o * 8, wl + b * 1024);
    }
    // Activations: 8 per thread per step; rows past the batch repeat its last
    // row (not stored). fp32 activations (xf) are rounded to bf16 (nearest
    // even) first, and the first expert block writes those bf16 rows to xb
    // for the expert kernels.
#pragma unroll
    for (int i = tid; i < TPB * kRouterKC / 8; i += NTH) {
        const int t = i / (kRouterKC / 8), kk = (i - t * (kRouterKC / 8)) * 8;
        const int tt = t < nb ? t : nb - 1;
        const size_t off = (size_t)(tb + tt) * H + c * kRouterKC + kk;
        uint4 v;
        if (xf) {
            const float4 lo = *reinterpret_cast<const float4*>(xf + off);
            const float4 hi = *reinterpret_cast<const float4*>(xf + off + 4);
            v = make_uint4(f32_to_bf16(lo.x) | (f32_to_bf16(lo.y) << 16),
                           f32_to_bf16(lo.z) | (f32_to_bf16(lo.w) << 16),
                           f32_to_bf16(hi.x) | (f32_to_bf16(hi.y) << 16),
                           f32_to_bf16(hi.z) | (f32_to_bf16(hi.w) << 16));
            if (blockIdx.y == 0 && t < nb) *reinterpret_cast<uint4*>(xb + off) = v;
        } else {
            v = *reinterpret_cast<const uint4*>(x + off);
        }
        const uint32_t xd[4] = {v.x, v.y, v.z, v.w};
        float4 lo, hi;
        lo.x = bf16_to_f32(xd[0] & 0xffffu); lo.y = __uint_as_float(xd[0] & 0xffff0000u);
        lo.z = bf16_to_f32(xd[1] & 0xffffu); lo.w = __uint_as_float(xd[1] & 0xffff0000u);
        hi.x = bf16_to_f32(xd[2] & 0xffffu); hi.y = __uint_as_float(xd[2] & 0xffff0000u);
        hi.z = bf16_to_f32(xd[3] & 0xffffu); hi.w = __uint_as_float(xd[3] & 0xffff0000u);
        *reinterpret_cast<float4*>(&xl[t][kk]) = lo;
        *reinterpret_cast<float4*>(&xl[t][kk + 4]) = hi;
    }
    wait_vmcnt<0>();
    __syncthreads();
    const int t0 = wave * NT, nt = min(NT, nb - t0);   // this wave's tokens
    if (nt <= 0) return;   // wave-uniform; no barrier follows
    uint4 wv[kRouterKC / 8];
#pragma unroll
    for (int j = 0; j < kRouterKC / 8; ++j)
        wv[j] = *reinterpret_cast<const uint4*>(wl + lane * 256 + ((j ^ (lane & 15)) << 4));
    const float* xw = &xl[t0][0];
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    // Step j: the 8 activations of every token (LDS broadcasts: every lane
    // reads the same bytes), read one step ahead; rows past nt repeat the
    // wave's last row.
    auto rd = [&](int j, float4 (&xv)[NT][2]) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int tt = t < nt ? t : nt - 1;
            xv[t][0] = *reinterpret_cast<const float4*>(xw + tt * kRouterKC + j * 8);
            xv[t][1] = *reinterpret_cast<const float4*>(xw + tt * kRouterKC + j * 8 + 4);
        }
    };
    float4 xs0[NT][2], xs1[NT][2];
    rd(0, xs0);
#pragma unroll
    for (int j = 0; j < kRouterKC / 8; ++j) {
        float4 (&cur)[NT][2] = (j & 1) ? xs1 : xs0;
        float4 (&nxt)[NT][2] = (j & 1) ? xs0 : xs1;
        if (j + 1 < kRouterKC / 8) rd(j + 1, nxt);
        const uint32_t wd[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
        float wf[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            wf[2 * q] = bf16_to_f32(wd[q] & 0xffffu);
            wf[2 * q + 1] = __uint_as_float(wd[q] & 0xffff0000u);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            acc[t] = __builtin_fmaf(cur[t][0].x, wf[0], acc[t]);
            acc[t] = __builtin_fmaf(cur[t][0].y, wf[1], acc[t]);
            acc[t] = __builtin_fmaf(cur[t][0].z, wf[2], acc[t]);
            acc[t] = __builtin_fmaf(cur[t][0].w, wf[3], acc[t]);
            acc[t] = __builtin_fmaf(cur[t][1].x, wf[4], acc[t]);
            acc[t] = __builtin_fmaf(cur[t][1].y, wf[5], acc[t]);
            acc[t] = __builtin_fmaf(cur[t][1].z, wf[6], acc[t]);
            acc[t] = __builtin_fmaf(cur[t][1].w, wf[7], acc[t]);
        }
        // Pin each step's chains here (otherwise the reads of later steps
        // are hoisted and the arithmetic sunk).
#pragma unroll
        for (int t = 0; t < NT; ++t) asm volatile("" : "+v"(acc[t]));
        __builtin_amdgcn_sched_barrier(0);
    }
    if (e < E) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
            if (t < nt) part[((size_t)c * n + tb + t0 + t) * E + e] = acc[t];
    }
    if (xsum && blockIdx.y == 0 && lane < nt) {
        float xs = 0.0f;
        for (int k = 0; k < kRouterKC; ++k) xs += xw[lane * kRouterKC + k];
        xsum[(size_t)(tb + t0 + lane) * nchunks + c] = xs;
    }
}

constexpr int kFoldThreads = 512;   // dispatch_block needs 8 waves

template <int NJ>
__global__ __launch_bounds__(kFoldThreads) void router_fold_select_kernel(
    const float* __restrict__ part, int nchunks, const float* __restrict__ e_bias, int n, int E,
    int topk, int norm_topk, float routed_scale, float* __restrict__ logits, int* __restrict__ ids,
    float* __restrict__ w, unsigned int* __restrict__ ticket, DispOut d) {
    __shared__ float lt[64 * NJ];
    __shared__ uint32_t tscratch[kTopkScratch];
    __shared__ int sids[8];
    __shared__ int last;
    __shared__ int dlds[dispatch_lds_ints<kFoldThreads>()];
    const int t = blockIdx.x;
    const size_t stride = (size_t)n * E;
    for (int e = threadIdx.x; e < E; e += kFoldThreads) {
        const float* p = part + (size_t)t * E + e;
        // Up to 48 partials in flight (one round trip at H = 6144), added in
        // chunk order.
        float total = 0.0f;
        for (int c = 0; c < nchunks; c += 48) {
            float v[48];
#pragma unroll
            for (int u = 0; u < 48; ++u) v[u] = p[min(c + u, nchunks - 1) * stride];
            const int m = min(48, nchunks - c);
            if (m == 48) {
#pragma unroll
                for (int u = 0; u < 48; ++u) total = total + v[u];
            } else {
#pragma unroll
                for (int u = 0; u < 48; ++u)
                    if (u < m) total = total + v[u];
            }
        }
        logits[(size_t)t * E + e] = total;
        lt[e] = total;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        // With a ticket the ids also go out with device-coherent stores (the
        // same values): the last workgroup to finish reads every token's ids
        // with coherent loads and dispatches.
        topk_wave_nj<false, NJ>(lt, e_bias, E, topk, norm_topk, routed_scale,
                                ids + (size_t)t * topk, w + (size_t)t * topk, tscratch, nullptr,
                                nullptr, ticket ? sids : nullptr);
        if (ticket) {
            if (threadIdx.x < topk) st_dev(ids + (size_t)t * topk + threadIdx.x, sids[threadIdx.x]);
            drain_vm();
            if (threadIdx.x == 0) last = ticket_dev(ticket) == (unsigned int)(n - 1);
        }
    }
    if (!ticket) return;
    __syncthreads();
    if (!last) return;   // workgroup-uniform
    dispatch_block<kFoldThreads, true>(ids, n, topk, E, d, dlds);
}

bool router_gemv_path(int n, int H, int E, int topk) {
    return n >= kGemvMinTokens && router_small_path(n, H, E, topk);
}

bool router_small_path(int n, int H, int E, int topk) {
    return n < kTiledMinTokens && H % kRouterKC == 0 && H / kRouterKC <= kSmallMaxChunks &&
           E <= 64 * kMaxPerLane && topk <= 8;
}

// K splits of the MFMA router pass: enough (up to 8) for about 512
// workgroups, two per CU (a batch of a few hundred tokens has only a few
// dozen 64 x 64 tiles; at 4096 tokens two splits measured 61 -> 46 us for
// this pass, +4 us for the refinement's extra reads).
int router_mfma_splits(int n, int E) {
    const long tiles = (long)((E + kMfmaExp - 1) / kMfmaExp) * ((n + kMfmaTok - 1) / kMfmaTok);
    int z = 1;
    while (z < 8 && tiles * z * 2 <= 512) z *= 2;
    return z;
}

size_t router_select_scratch_bytes(int n, int H, int E) {
    const size_t a = router_logits_scratch_bytes(n, H, E);
    // The MFMA pass: S partials [nsplit][n][E], L~ partials of splits 1.. .
    const int z = n >= kTiledMinTokens ? router_mfma_splits(n, E) : 1;
    const size_t b = (size_t)(2 * z - 1) * n * E * 4;
    // Small batches: the order codes and scores; from kGemvMinTokens the
    // chunk partials [H / 128][n][E] instead.
    size_t c = (size_t)n * E * 4 * 2;
    // (+ 256 bytes: the fold kernel's ticket.)
    if (n >= kGemvMinTokens && n < kTiledMinTokens && (size_t)(H / kRouterKC) * n * E * 4 + 256 > c)
        c = (size_t)(H / kRouterKC) * n * E * 4 + 256;
    const size_t m = a > b ? a : b;
    return m > c ? m : c;
}

int launch_router_select(const uint16_t* x, const uint16_t* wr, const float* e_bias, int n, int H,
                         int E, int topk, int norm_topk, float routed_scale, float* logits,
                         float* xsum, float* scratch, int* ids, float* w, hipStream_t s,
                         const DispOut* disp, bool* dispatched, bool select, const float* xf,
                         uint16_t* xb, uint16_t* xh, float* xrho, bool* x16_done) {
    const int nchunks = H / kRouterKC;
    if (dispatched) *dispatched = false;
    if (xf && !router_small_path(n, H, E, topk)) return -2;   // the caller converts x first
    if (select && router_gemv_path(n, H, E, topk)) {
        const size_t need = (size_t)nchunks * n * E * 4 + 256;
        if (!scratch || router_select_scratch_bytes(n, H, E) < need) return -3;
        // With the dispatch outputs the last fold workgroup dispatches too.
        const bool dd = disp && E <= kDispMaxE;
        unsigned int* ticket = dd ? reinterpret_cast<unsigned int*>(scratch + (size_t)nchunks * n * E)
                                  : nullptr;
        // Tokens per wave: 2 up to 16 tokens (more workgroups to fill the
        // CUs), else 4 (measured per layer at 16 / 32 / 64 / 128 tokens: 8
        // was 1-5 us slower, its workgroups stacking two to a CU).
        const int NT = n <= 16 ? 2 : 4;
        dim3 grid((unsigned)nchunks, (unsigned)((E + 63) / 64),
                  (unsigned)((n + kGemvWaves * NT - 1) / (kGemvWaves * NT)));
        auto gemv = NT == 2 ? router_gemv_kernel<2> : router_gemv_kernel<4>;
        hipLaunchKernelGGL(gemv, grid, dim3(64 * kGemvWaves), 0, s, x, wr, n, H, E, scratch, xsum,
                           ticket, xf, xb);
        if (hipGetLastError() != hipSuccess) return -4;
        auto fold = E <= 64 ? router_fold_select_kernel<1> : E <= 128 ? router_fold_select_kernel<2>
                                   : E <= 256 ? router_fold_select_kernel<4> : router_fold_select_kernel<8>;
        hipLaunchKernelGGL(fold, dim3((unsigned)n), dim3(kFoldThreads), 0, s, scratch, nchunks,
                           e_bias, n, E, topk, norm_topk, routed_scale, logits, ids, w, ticket,
                           dd ? *disp : DispOut{});
        if (hipGetLastError() != hipSuccess) return -4;
        if (dispatched) *dispatched = dd;
        return 0;
    }
    if (router_small_path(n, H, E, topk)) {
        // scratch: the order codes and scores [2][n][E] handed to the top-k.
        if (!scratch || router_select_scratch_bytes(n, H, E) < (size_t)2 * n * E * 4) return -3;
        // Experts per workgroup: as few as fill every CU once (one round of
        // workgroups; with fewer experts per workgroup each thread runs
        // fewer tokens), as many as keep a second round away.
        static int cus = 0;
        if (!cus) {
            int dev = 0;
            cus = 256;
            if (hipGetDevice(&dev) == hipSuccess)
                (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        }
        const int ntg = (n + kRouterTG - 1) / kRouterTG;
        // (One token group included: one expert per workgroup at E = 256 on
        // 256 CUs measured faster than two, 4.9 against 5.3 us at one token.)
        int epw = (E * ntg + cus - 1) / cus;
        if (epw > kSmallThreads / nchunks) epw = kSmallThreads / nchunks;
        if (epw < 1) epw = 1;
        int slices = 1;
        while (slices < kRouterTG && 2 * slices * epw * nchunks <= kSmallThreads) slices *= 2;
        const bool dd = disp && E <= kDispMaxE;
        dim3 grid((unsigned)((E + epw - 1) / epw), (unsigned)((n + kRouterTG - 1) / kRouterTG));
        const size_t lds = (size_t)small_x_bytes(nchunks) + (size_t)epw * nchunks * kRouterTG * 4;
        static bool attr_set = false;
        if (!attr_set) {
            if (hipFuncSetAttribute(reinterpret_cast<const void*>(&router_small_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    small_x_bytes(kSmallMaxChunks) +
                                        kSmallThreads * kRouterTG * 4) != hipSuccess)
                return -4;
            attr_set = true;
        }
        hipLaunchKernelGGL(router_small_kernel, grid, dim3(kSmallThreads), lds, s, x, wr, e_bias, n,
                           H, E, epw, logits, xsum, slices, reinterpret_cast<uint32_t*>(scratch),
                           select ? nullptr : disp->zero, select ? 0 : disp->nzero, xf, xb);
        if (hipGetLastError() != hipSuccess) return -4;
        if (!select) return 0;   // codes and scores only: the gate/up kernel selects
        // Selection: one workgroup (and then the dispatch too) up to
        // kFinishDispMax tokens, else one wave per token.
        const bool one = n <= kFinishDispMax;
        const unsigned fg = one ? 1u : (unsigned)((n + kSmallThreads / 64 - 1) / (kSmallThreads / 64));
        auto fin = E <= 64 ? router_finish_kernel<1> : E <= 128 ? router_finish_kernel<2>
                                     : E <= 256 ? router_finish_kernel<4> : router_finish_kernel<8>;
        hipLaunchKernelGGL(fin, dim3(fg), dim3(kSmallThreads), 0, s, logits, e_bias, n, E, topk,
                           norm_topk, routed_scale, ids, w, reinterpret_cast<const uint32_t*>(scratch),
                           dd && one ? *disp : DispOut{}, dd && one ? 1 : 0);
        if (hipGetLastError() != hipSuccess) return -4;
        if (dispatched) *dispatched = dd && one;
        return 0;
    }
    if (n >= kTiledMinTokens && H % kMfmaK == 0 && H % kRouterKC == 0 && nchunks <= 64 &&
        E <= 64 * kMaxPerLane) {
        if (!scratch) return -3;
        const int nsplit = router_mfma_splits(n, E);
        dim3 grid((unsigned)((E + kMfmaExp - 1) / kMfmaExp), (unsigned)((n + kMfmaTok - 1) / kMfmaTok),
                  (unsigned)nsplit);
        hipLaunchKernelGGL(router_mfma_kernel, grid, dim3(256), kMfmaD * 2 * kMfmaTok * 128, s, x,
                           wr, n, H, E, logits, scratch, scratch + (size_t)nsplit * n * E, nsplit);
        if (hipGetLastError() != hipSuccess) return -4;
        if (n < kRefineSplitMax) {
            auto refine = E <= 64 ? router_refine_kernel<1, kRefineSplit>
                        : E <= 128 ? router_refine_kernel<2, kRefineSplit>
                        : E <= 256 ? router_refine_kernel<4, kRefineSplit>
                                   : router_refine_kernel<8, kRefineSplit>;
            hipLaunchKernelGGL(refine, dim3((unsigned)n), dim3(kRefineSplit * 64), 0, s, x, wr, e_bias,
                               scratch, n, H, E, topk, logits, xsum, nsplit, xh, xrho);
        } else {
            auto refine = E <= 64 ? router_refine_kernel<1, 1> : E <= 128 ? router_refine_kernel<2, 1>
                        : E <= 256 ? router_refine_kernel<4, 1> : router_refine_kernel<8, 1>;
            hipLaunchKernelGGL(refine, dim3((unsigned)((n + kRefineWaves - 1) / kRefineWaves)),
                               dim3(kRefineWaves * 64), 0, s, x, wr, e_bias, scratch, n, H, E, topk,
                               logits, xsum, nsplit, xh, xrho);
        }
        if (hipGetLastError() != hipSuccess) return -4;
        if (x16_done) *x16_done = xh && xrho;
    } else {
        const int rc = launch_router_logits(x, wr, n, H, E, logits, xsum, scratch, s);
        if (rc) return rc;
    }
    return launch_router_topk(logits, e_bias, n, E, topk, norm_topk, routed_scale, ids, w, s);
}

// ---------------------------------------------------------------------------
// fp32 activations and router weights (gemm_fp32's arguments, the
// reference's router call gemm_linear(s.normed, d.router, ...),
// src/model_gpu.cpp:1448, cuda/kernels.cuh:37-38): both are rounded to bf16
// (round-to-nearest-even, as the bf16 entry's callers round them) on load,
// then the same fixed order as the bf16 path: per 128-K chunk an ascending-K
// fma chain from zero, chunk partials added in chunk order; then + bias[e]
// (nullable). No workspace: grid (ceil(E / epw), ceil(n / 8)) of 512
// threads, thread (expert el, chunk c) for every token of its group of 8.
// LDS: the group's activations as bf16 rows R = t * nchunks + c of 256 B,
// 16-B piece o at slot o ^ (R & 15) (threads of consecutive chunks reading
// the same piece hit distinct banks), then the partials [pair][token].
constexpr int kF32Threads = 512;

__host__ __device__ constexpr size_t f32_router_lds(int H, int epw) {
    return (size_t)kRouterTG * H * 2 + (size_t)epw * (H / kRouterKC) * kRouterTG * 4;
}

__global__ __launch_bounds__(kF32Threads) void router_logits_f32_kernel(
    const float* __restrict__ x, const float* __restrict__ W, const float* __restrict__ bias,
    float* __restrict__ y, int n, int H, int E, int epw) {
    extern __shared__ __align__(16) char f32_lds[];
    const int nchunks = H / kRouterKC;
    const int tid = threadIdx.x;
    const int t0 = blockIdx.y * kRouterTG, nt = min(kRouterTG, n - t0);
    char* xl = f32_lds;
    float* part = reinterpret_cast<float*>(f32_lds + (size_t)kRouterTG * H * 2);
    // Stage: 8 consecutive K of one row per thread step (one 16-B piece).
    const int pieces = nt * (H / 8);
    for (int i = tid; i < pieces; i += kF32Threads) {
        const int t = i / (H / 8), kp = i - t * (H / 8);
        const int c = kp / (kRouterKC / 8), o = kp % (kRouterKC / 8);
        const float4* src = reinterpret_cast<const float4*>(x + (size_t)(t0 + t) * H + kp * 8);
        const float4 a = src[0], b = src[1];
        uint4 v;
        v.x = f32_to_bf16(a.x) | (f32_to_bf16(a.y) << 16);
        v.y = f32_to_bf16(a.z) | (f32_to_bf16(a.w) << 16);
        v.z = f32_to_bf16(b.x) | (f32_to_bf16(b.y) << 16);
        v.w = f32_to_bf16(b.z) | (f32_to_bf16(b.w) << 16);
        const int R = t * nchunks + c;
        *reinterpret_cast<uint4*>(xl + R * 256 + ((o ^ (R & 15)) << 4)) = v;
    }
    const int pair = tid, el = pair / nchunks, c = pair - el * nchunks;
    const int e = blockIdx.x * epw + el;
    const bool active = pair < epw * nchunks && e < E;
    uint4 wv[kRouterKC / 8];
    if (active) {
        const float4* wp = reinterpret_cast<const float4*>(W + (size_t)e * H + c * kRouterKC);
#pragma unroll
        for (int j = 0; j < kRouterKC / 8; ++j) {
            const float4 a = wp[2 * j], b = wp[2 * j + 1];
            wv[j].x = f32_to_bf16(a.x) | (f32_to_bf16(a.y) << 16);
            wv[j].y = f32_to_bf16(a.z) | (f32_to_bf16(a.w) << 16);
            wv[j].z = f32_to_bf16(b.x) | (f32_to_bf16(b.y) << 16);
            wv[j].w = f32_to_bf16(b.z) | (f32_to_bf16(b.w) << 16);
        }
    }
    __syncthreads();
    if (active) {
        for (int t = 0; t < nt; ++t) {
            const int R = t * nchunks + c;
            const char* row = xl + R * 256;
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < kRouterKC / 8; ++j) {
                const uint4 xv = *reinterpret_cast<const uint4*>(row + ((j ^ (R & 15)) << 4));
                const uint32_t xd[4] = {xv.x, xv.y, xv.z, xv.w};
                const uint32_t wd[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    acc = __builtin_fmaf(bf16_to_f32(xd[q] & 0xffffu), bf16_to_f32(wd[q] & 0xffffu), acc);
                    acc = __builtin_fmaf(__uint_as_float(xd[q] & 0xffff0000u),
                                         __uint_as_float(wd[q] & 0xffff0000u), acc);
                }
            }
            part[pair * kRouterTG + t] = acc;
        }
    }
    __syncthreads();
    if (tid < epw * kRouterTG) {
        const int el2 = tid / kRouterTG, t = tid % kRouterTG;
        const int e2 = blockIdx.x * epw + el2;
        if (e2 < E && t < nt) {
            const float total = chunk_sum(part + el2 * nchunks * kRouterTG + t, kRouterTG, nchunks);
            y[(size_t)(t0 + t) * E + e2] = bias ? total + bias[e2] : total;
        }
    }
}

int launch_router_logits_f32(const float* x, const float* W, const float* bias, float* y, int n,
                             int H, int E, hipStream_t s) {
    if (H % kRouterKC || H / kRouterKC > kF32Threads || H > 8192) return -2;
    const int nchunks = H / kRouterKC;
    const int epw = kF32Threads / nchunks;
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&router_logits_f32_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)f32_router_lds(8192, kF32Threads / (8192 / kRouterKC))) != hipSuccess)
            return -4;
        attr_set = true;
    }
    dim3 grid((unsigned)((E + epw - 1) / epw), (unsigned)((n + kRouterTG - 1) / kRouterTG));
    hipLaunchKernelGGL(router_logits_f32_kernel, grid, dim3(kF32Threads), f32_router_lds(H, epw), s, x, W,
                       bias, y, n, H, E, epw);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

size_t router_logits_scratch_bytes(int n, int H, int E) {
    if (n >= kTiledMinTokens && H % kRouterKC == 0) return 0;
    return (size_t)n * ((H + kRouterKC - 1) / kRouterKC) * E * 4;
}

int launch_router_logits(const uint16_t* x, const uint16_t* wr, int n, int H, int E,
                         float* logits, float* xsum, float* scratch, hipStream_t s) {
    const int nchunks = (H + kRouterKC - 1) / kRouterKC;
    if (nchunks > kRouterMaxChunks) return -2;
    if (n >= kTiledMinTokens && H % kRouterKC == 0) {
        const long blocks = (long)((E + kTiledExp - 1) / kTiledExp) * ((n + kTiledTok - 1) / kTiledTok);
        hipLaunchKernelGGL(router_logits_tiled_kernel, dim3((unsigned)blocks), dim3(kTiledThreads),
                           0, s, x, wr, n, H, E, logits);
    } else {
        if (!scratch) return -3;
        const long blocks = (long)nchunks * ((E + 63) / 64) * ((n + kRouterTG - 1) / kRouterTG);
        hipLaunchKernelGGL(router_partials_kernel, dim3((unsigned)blocks), dim3(64), 0, s, x, wr,
                           n, H, E, scratch, H % kRouterKC == 0 ? xsum : nullptr);
        if (hipGetLastError() != hipSuccess) return -4;
        const long outs = (long)n * E;
        hipLaunchKernelGGL(router_fold_kernel, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0,
                           s, scratch, n, nchunks, E, logits);
    }
    if (hipGetLastError() != hipSuccess) return -4;
    const bool small = !(n >= kTiledMinTokens && H % kRouterKC == 0);
    return xsum && !small ? launch_xsum(x, n, H, xsum, s) : 0;
}

int launch_xsum(const uint16_t* x, int n, int H, float* xsum, hipStream_t s) {
    const long items = (long)n * (H / kRouterKC);
    hipLaunchKernelGGL(xsum_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, s, x,
                       n, H, xsum);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_router_topk(const float* logits, const float* e_bias, int n, int E, int topk,
                       int norm_topk, float routed_scale, int* ids, float* w, hipStream_t s) {
    hipLaunchKernelGGL(router_topk_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s,
                       logits, e_bias, n, E, topk, norm_topk, routed_scale, ids, w);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace glmmoe
