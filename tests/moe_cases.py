"""Synthetic MoE layers of the benchmark shapes, shared by tests, smoke and bench.

Layers are generated in the REFERENCE weight layout (cuda/kernels.cuh:259-268:
packed int4 [rows, K/2], low nibble = even column, value = nibble - 8; scales
[rows, K/128]) and packed to the native layout on the device by the library.
Values follow the benchmark definition: int4 codes uniform over [-8, 7],
scales |N(0, 0.01)| in bf16, router weights bf16 N(0, 0.02), correction bias
U(-0.1, 0.1), activations bf16 N(0, 1).
"""
import os

import numpy as np
import torch

# Host threads for the oracle's row-batched expert FFN (the GPU box gives a
# process a 16-CPU share whatever os.cpu_count() reports).
ORACLE_THREADS = max(1, min(16, os.cpu_count() or 1))


def bf16_bits(a):
    """fp32 numpy -> bf16 bit patterns (round to nearest even)."""
    a = np.ascontiguousarray(a, np.float32)
    b = a.view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return b.astype(np.uint16)


def bits_to_f32(u16):
    return (np.ascontiguousarray(u16, np.uint16).astype(np.uint32) << 16).view(np.float32)


def zipf_log_prior(E, s, gen):
    """log-prior -s*ln(rank+1) over a seeded permutation of the experts."""
    perm = torch.randperm(E, generator=gen, device="cpu")
    rank = torch.empty(E, dtype=torch.float32)
    rank[perm] = torch.arange(E, dtype=torch.float32)
    return -s * torch.log(rank + 1.0)


class SynthLayer:
    """A W4A16 MoE layer generated on the GPU from a seed (reference layout kept
    for the oracle), plus its packed device form."""

    def __init__(self, H, E, k, I, seed=0, shared=True, zipf_s=None, device="cuda",
                 norm_topk=True, routed_scale=2.5, down_scale_mul=1.0):
        from glmserve_amd import W4A16MoELayer, pack_w4a16
        self.H, self.E, self.k, self.I = H, E, k, I
        self.norm_topk, self.routed_scale = norm_topk, routed_scale
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        gc = torch.Generator(device="cpu")
        gc.manual_seed(seed + 7)
        dev = device
        self.router_w = (0.02 * torch.randn(E, H, generator=g, device=dev)).to(torch.bfloat16)
        bias = (torch.rand(E, generator=gc) * 0.2 - 0.1)
        if zipf_s is not None:
            bias = bias + zipf_log_prior(E, zipf_s, gc)
        self.e_bias = bias.to(torch.float32).to(dev)

        def mat(n, rows, K):
            q = torch.randint(0, 256, (n, rows, K // 2), generator=g, device=dev, dtype=torch.uint8)
            s = (0.01 * torch.randn(n, rows, K // 128, generator=g, device=dev)).abs().to(torch.bfloat16)
            return q, s

        def scaled(m):
            # down_scale_mul: every down scale times a factor (rounded to bf16
            # again), for scales outside the usual magnitude.
            if down_scale_mul == 1.0:
                return m
            return m[0], (m[1].float() * down_scale_mul).to(torch.bfloat16)

        self.gate = mat(E, I, H)
        self.up = mat(E, I, H)
        self.down = scaled(mat(E, H, I))
        self.shared = (mat(1, I, H), mat(1, I, H), scaled(mat(1, H, I))) if shared else None
        self.has_shared_expert = shared
        pk = lambda m, rows, K: pack_w4a16(m[0], m[1], m[0].shape[0], rows, K)
        sh_packed = None
        if shared:
            sh_packed = (pk(self.shared[0], I, H), pk(self.shared[1], I, H), pk(self.shared[2], H, I))
        self.layer = W4A16MoELayer(H, I, E, k, self.router_w, self.e_bias, pk(self.gate, I, H),
                                   pk(self.up, I, H), pk(self.down, H, I), sh_packed,
                                   norm_topk=norm_topk, routed_scale=routed_scale)

    def x(self, n, seed):
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        return torch.randn(n, self.H, generator=g, device="cuda").to(torch.bfloat16)

    # ---- oracle side (host) -------------------------------------------------
    def dequant_expert(self, oracle, e):
        """fp32 (gate, up, down) of routed expert e (or the shared one for e == E)."""
        mats = self.shared if e == self.E else (self.gate, self.up, self.down)
        idx = 0 if e == self.E else e
        out = []
        for (q, s), (rows, K) in zip(mats, [(self.I, self.H), (self.I, self.H), (self.H, self.I)]):
            qn = q[idx].cpu().numpy()
            sn = s[idx].float().cpu().numpy()
            out.append(oracle.dequant_int4_rows(qn, sn, K, 128))
        return out

    def oracle_forward(self, oracle, x_bf16, tokens, logits, nthreads=8):
        """Oracle layer output for the given token indices, with the given logits
        (routing redone by the oracle from them). Materializes only the experts
        those tokens select."""
        xf = bits_to_f32(x_bf16[tokens].view(torch.int16).cpu().numpy().view(np.uint16))
        lg = np.ascontiguousarray(logits[tokens], np.float32)
        eb = self.e_bias.cpu().numpy()
        ids, _ = oracle.router_topk(lg, eb, self.k, self.norm_topk, self.routed_scale)
        need = sorted(set(ids.ravel().tolist()))
        gate = [None] * self.E
        up = [None] * self.E
        down = [None] * self.E
        for e in need:
            gate[e], up[e], down[e] = self.dequant_expert(oracle, e)
        sh = self.dequant_expert(oracle, self.E) if self.shared is not None else None
        return oracle.moe_forward(xf, self.E, self.k, gate, up, down, sh, logits=lg, e_bias=eb,
                                  norm_topk=self.norm_topk, routed_scale=self.routed_scale,
                                  nthreads=nthreads)


def _oracle_full(L, oracle, xf, ids, w, h_fp8):
    """Every token's oracle output for the given routing, experts materialized
    one at a time (oracle.moe_forward_streamed)."""
    sh = L.dequant_expert(oracle, L.E) if L.has_shared_expert else None
    return oracle.moe_forward_streamed(xf, ids, w, lambda e: L.dequant_expert(oracle, e), sh,
                                       h_fp8=h_fp8, nthreads=ORACLE_THREADS)


def oracle_full_w4(L, oracle, x_bf16, ids, w):
    """Oracle output of every token of a W4A16 layer for routing (ids, w)."""
    xf = bits_to_f32(x_bf16.view(torch.int16).cpu().numpy().view(np.uint16))
    return _oracle_full(L, oracle, xf, ids, w, h_fp8=False)


def rel_err(got, ref):
    """max|got - ref| / max|ref|: the reference's tests/test_qgemm.cpp:17-26
    check() without its max(1, .) floor, which would make small-magnitude
    layers pass on absolute error alone."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(1e-30, float(np.max(np.abs(ref)))))


class SynthFp8Layer:
    """An FP8 MoE layer (configs[4] format) generated on the GPU from a seed.

    Each matrix is e4m3 codes [rows, K] with fp32 scales per 128 x 128 block:
    codes are e4m3(clamp(N(0,1) * 96, +-448)) (round to nearest even by torch's
    float8_e4m3fn conversion; never the NaN codes), block scales
    0.02 / 96 * U(0.5, 1.5), so weights are ~N(0, 0.02) with per-block spread.
    Every (matrix, expert) has its own seed, so the oracle side regenerates the
    experts it needs instead of keeping a host copy of all of them."""

    def __init__(self, H, E, k, I, seed=0, shared=True, zipf_s=None, device="cuda",
                 norm_topk=True, routed_scale=2.5):
        from glmserve_amd import FP8MoELayer, lib, pack_fp8
        self.H, self.E, self.k, self.I, self.seed = H, E, k, I, seed
        self.norm_topk, self.routed_scale = norm_topk, routed_scale
        self.has_shared = shared
        self.has_shared_expert = shared
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        gc = torch.Generator(device="cpu")
        gc.manual_seed(seed + 7)
        self.router_w = (0.02 * torch.randn(E, H, generator=g, device=device)).to(torch.bfloat16)
        bias = (torch.rand(E, generator=gc) * 0.2 - 0.1)
        if zipf_s is not None:
            bias = bias + zipf_log_prior(E, zipf_s, gc)
        self.e_bias = bias.to(torch.float32).to(device)
        shapes = [(I, H), (I, H), (H, I)]
        self.packed, self.scales = [], []
        for m, (rows, K) in enumerate(shapes):
            nm = E + (1 if shared else 0)
            pq = torch.empty(nm * lib().glmmoe_fp8_packed_bytes(rows, K), dtype=torch.uint8,
                             device=device)
            sc = torch.empty(nm, rows // 128, K // 128, dtype=torch.float32, device=device)
            per = rows * K
            for e in range(nm):
                q, s = self.matrix(m, e)
                pack_fp8(q, 1, rows, K, out=pq[e * per:(e + 1) * per])
                sc[e] = s
            self.packed.append(pq)
            self.scales.append(sc)
        torch.cuda.synchronize()
        per = [r * K for r, K in shapes]
        routed = [(self.packed[m][:E * per[m]], self.scales[m][:E]) for m in range(3)]
        sh = None
        if shared:
            sh = tuple((self.packed[m][E * per[m]:], self.scales[m][E:]) for m in range(3))
        self.layer = FP8MoELayer(H, I, E, k, self.router_w, self.e_bias, routed[0], routed[1],
                                 routed[2], sh, norm_topk=norm_topk, routed_scale=routed_scale)

    def matrix(self, m, e, device="cuda"):
        """(codes uint8 [rows, K], scales fp32 [rows/128, K/128]) of matrix m
        (0 gate, 1 up, 2 down) of expert e (e == E: the shared expert)."""
        rows, K = [(self.I, self.H), (self.I, self.H), (self.H, self.I)][m]
        g = torch.Generator(device=device)
        g.manual_seed(self.seed * 1000003 + e * 3 + m + 1)
        v = (torch.randn(rows, K, generator=g, device=device) * 96.0).clamp_(-448.0, 448.0)
        q = v.to(torch.float8_e4m3fn).view(torch.uint8)
        s = (0.02 / 96.0) * (0.5 + torch.rand(rows // 128, K // 128, generator=g, device=device))
        return q, s.to(torch.float32)

    def x(self, n, seed):
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        return torch.randn(n, self.H, generator=g, device="cuda").to(torch.bfloat16)

    def dequant_expert(self, oracle, e):
        out = []
        for m in range(3):
            q, s = self.matrix(m, e)
            out.append(oracle.dequant_e4m3_blocks(q.cpu().numpy(), s.cpu().numpy()))
        return out

    def oracle_forward(self, oracle, x_bf16, tokens, logits, nthreads=8):
        """Oracle output for the given tokens: x quantized per token and 128
        channels (oracle rule) and dequantized, h quantized the same way."""
        xf = bits_to_f32(x_bf16[tokens].view(torch.int16).cpu().numpy().view(np.uint16))
        q, s = oracle.quant_act_e4m3(xf)
        dec = np.array([oracle.e4m3_to_f32(c) for c in range(256)], np.float32)
        xd = (dec[q].reshape(len(tokens), -1, 128) * s[:, :, None]).reshape(len(tokens), self.H)
        lg = np.ascontiguousarray(logits[tokens], np.float32)
        eb = self.e_bias.cpu().numpy()
        ids, _ = oracle.router_topk(lg, eb, self.k, self.norm_topk, self.routed_scale)
        need = sorted(set(ids.ravel().tolist()))
        gate, up, down = [None] * self.E, [None] * self.E, [None] * self.E
        for e in need:
            gate[e], up[e], down[e] = self.dequant_expert(oracle, e)
        sh = self.dequant_expert(oracle, self.E) if self.has_shared else None
        return oracle.moe_forward(xd, self.E, self.k, gate, up, down, sh, logits=lg, e_bias=eb,
                                  norm_topk=self.norm_topk, routed_scale=self.routed_scale,
                                  nthreads=nthreads, h_fp8=True)


def oracle_full_fp8(L, oracle, x_bf16, ids, w):
    """Oracle output of every token of an FP8 layer for routing (ids, w): x
    quantized per token and 128 channels and dequantized, h quantized the
    same way (SynthFp8Layer.oracle_forward's rule)."""
    xf = bits_to_f32(x_bf16.view(torch.int16).cpu().numpy().view(np.uint16))
    q, s = oracle.quant_act_e4m3(xf)
    dec = np.array([oracle.e4m3_to_f32(c) for c in range(256)], np.float32)
    n = xf.shape[0]
    xd = (dec[q].reshape(n, -1, 128) * s[:, :, None]).reshape(n, L.H)
    return _oracle_full(L, oracle, xd, ids, w, h_fp8=True)


# GGUF types with block geometry (elements, bytes) and the byte offsets of
# their fp16 scale fields (src/gguf_quant.cpp:98-262; 0 = F32, 1 = F16).
GGUF_TYPES = {0: (1, 4, ()), 1: (1, 2, ()), 8: (32, 34, (0,)), 11: (256, 110, (108,)),
              12: (256, 144, (0, 2)), 13: (256, 176, (0, 2)), 14: (256, 210, (208,)),
              18: (256, 98, (0,)), 23: (256, 136, (0,))}


def random_gguf_rows(qtype, rows, n, rng, scale=1e-2):
    """rows x n elements of GGUF type qtype as uint8 [rows, row_bytes]: random
    codes with finite fp16 scales of about `scale` (random bytes there could be
    Inf / NaN)."""
    be, bb, dofs = GGUF_TYPES[qtype]
    nb = n // be
    if qtype == 0:
        return rng.standard_normal((rows, n)).astype(np.float32).view(np.uint8)
    if qtype == 1:
        return (rng.standard_normal((rows, n)) * 0.1).astype(np.float16).view(np.uint8)
    data = rng.integers(0, 256, (rows, nb, bb), dtype=np.uint8)
    d = (rng.uniform(0.5, 1.5, (rows, nb, len(dofs))) * scale).astype(np.float16).view(np.uint8)
    for i, o in enumerate(dofs):
        data[:, :, o:o + 2] = d[:, :, 2 * i:2 * i + 2]
    return data.reshape(rows, nb * bb)
