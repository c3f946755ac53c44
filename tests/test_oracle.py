"""Pins the CPU oracle (oracle/moe_oracle.c) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the oracle (a dropped
term, a wrong sign or index, a transposed operand, a wrong tie rule) fails:
  * closed forms and exhaustive enumerations (bf16, e4m3, int4 nibbles);
  * brute force on small inputs (full sorts, fp64 dot products);
  * the compiled reference itself (oracle/_ref: GLM52Model::moe_mlp and
    dequant_int4_to_f32 built from the glmserve sources), where available.
The reference holds no golden vectors for this path (its MoE tests regenerate
inputs from std::mt19937 at run time), so these are the pins.
"""
import math

import numpy as np
import pytest

from moe_cases import bf16_bits, bits_to_f32


def _ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


# ---- exp / sigmoid / silu ---------------------------------------------------

def test_expf_accuracy_and_specials(oracle):
    xs = np.linspace(-80.0, 80.0, 20001, dtype=np.float32)
    got = np.array([oracle.expf(float(x)) for x in xs], np.float32)
    ref = np.exp(xs.astype(np.float64)).astype(np.float32)
    assert _ulp_diff(got, ref).max() <= 2
    assert oracle.expf(0.0) == 1.0
    assert oracle.expf(1.0) == np.float32(math.e) or _ulp_diff([oracle.expf(1.0)], [math.e])[0] <= 1
    assert math.isnan(oracle.expf(float("nan")))
    # Clamp: arguments beyond +-80 evaluate at +-80.
    assert oracle.expf(200.0) == oracle.expf(80.0)
    assert oracle.expf(-200.0) == oracle.expf(-80.0)


def test_sigmoid_silu(oracle):
    xs = np.linspace(-30, 30, 4001).astype(np.float32).astype(np.float64)   # exact f32 inputs
    for x in xs:
        s = oracle.sigmoid(float(x))
        assert abs(s - 1.0 / (1.0 + math.exp(-x))) <= 1e-6 * max(s, 1e-30) + 1e-38   # <= 8 ulp
        v = oracle.silu(float(x))
        assert abs(v - x / (1.0 + math.exp(-x))) <= 1e-6 * abs(v) + 1e-30
    assert oracle.sigmoid(0.0) == 0.5
    assert oracle.silu(0.0) == 0.0


# ---- bf16 -------------------------------------------------------------------

def test_bf16_decode_exhaustive(oracle):
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.bf16_to_f32(allb)
    assert np.array_equal(got.view(np.uint32), allb.astype(np.uint32) << 16)


def test_bf16_encode_rne(oracle):
    rng = np.random.default_rng(0)
    mag = (np.abs(rng.standard_normal(200000)) * 10.0 ** rng.integers(-30, 30, 200000)).astype(np.float32)
    mag = mag[(mag.view(np.uint32) >> 16) < 0x7F7F]        # below the largest finite bf16
    for x in (mag, -mag):
        got = oracle.f32_to_bf16(x).astype(np.int64)
        # The result is one of the two bf16 neighbours, the nearer one; ties to even.
        lo = (x.view(np.uint32) >> 16).astype(np.int64)
        flo = bits_to_f32(lo.astype(np.uint16)).astype(np.float64)
        fhi = bits_to_f32((lo + 1).astype(np.uint16)).astype(np.float64)
        xd = x.astype(np.float64)
        dlo, dhi = np.abs(xd - flo), np.abs(xd - fhi)
        want = np.where(dlo < dhi, lo, np.where(dhi < dlo, lo + 1, np.where(lo % 2 == 0, lo, lo + 1)))
        assert np.array_equal(got, want)
    # Exact ties: mantissa tail 0x8000 rounds to the even neighbour.
    ties = np.array([0x3F808000, 0x3F818000, 0xBF808000], np.uint32).view(np.float32)
    assert list(oracle.f32_to_bf16(ties)) == [0x3F80, 0x3F82, 0xBF80]


# ---- FP8 e4m3 -----------------------------------------------------------------

def test_e4m3_decode_exhaustive_vs_torch(oracle):
    torch = pytest.importorskip("torch")
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    for c in range(256):
        got = oracle.e4m3_to_f32(c)
        if c in (0x7F, 0xFF):   # OCP NaN; the reference decodes +-480 (include/common.hpp:182-200)
            assert got == (480.0 if c == 0x7F else -480.0)
        else:
            assert got == ref[c], c


def test_e4m3_encode_rne_vs_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-448, 448, 20000), rng.standard_normal(20000) * 0.01,
                        rng.standard_normal(2000) * 1e-4]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([oracle.f32_to_e4m3(float(v)) for v in x], np.uint8)
    # +-0 may differ only in sign for values that round to zero
    same = (got == ref) | (((got & 0x7F) == 0) & ((ref & 0x7F) == 0))
    assert same.all()
    # Saturation to +-448, never the NaN codes.
    assert oracle.f32_to_e4m3(1e6) == 0x7E and oracle.f32_to_e4m3(-1e6) == 0xFE
    assert oracle.f32_to_e4m3(460.0) == 0x7E


# ---- int4 -----------------------------------------------------------------------

def test_dequant_int4_exhaustive_vs_reference(oracle, ref):
    # Every byte value once (512 columns), four groups of 128 with different
    # scales (incl. negative and tiny).
    q = np.arange(256, dtype=np.uint8).reshape(1, 256)
    scales = np.array([[0.37, -2.5, 1e-30, 7.0]], np.float32)
    out = oracle.dequant_int4_rows(q, scales, 512, 128).ravel()
    assert np.array_equal(out, ref.dequant_int4(q.ravel(), scales.ravel(), 512, 128))
    # Closed form: low nibble = even column, zero point 8.
    vals = np.empty(512, np.float32)
    vals[0::2], vals[1::2] = q.ravel() & 0xF, q.ravel() >> 4
    assert np.array_equal(out, ((vals - 8) * np.repeat(scales.ravel(), 128)).astype(np.float32))


def test_quantize_w4_roundtrip(oracle):
    rng = np.random.default_rng(2)
    w = (0.02 * rng.standard_normal((32, 384))).astype(np.float32)
    w[3, :128] = 0.0                      # all-zero group -> scale 1.0
    q, s = oracle.quantize_w4_rows(w, 128)
    assert s[3, 0] == 1.0
    amax = np.abs(w.reshape(32, 3, 128)).max(axis=2)
    assert np.allclose(s[np.arange(32) != 3], (amax / 7.0)[np.arange(32) != 3], rtol=1e-7)
    back = oracle.dequant_int4_rows(q, s, 384, 128)
    err = np.abs(back - w).reshape(32, 3, 128).max(axis=2)
    # Values inside +-7s round to the nearest step; the clipped -8 step never
    # triggers for a symmetric absmax scale, so |err| <= s/2.
    assert (err <= s / 2 + 1e-12).all()


# ---- router ---------------------------------------------------------------------

def test_router_logits_exact_on_integers(oracle):
    rng = np.random.default_rng(3)
    for n, H, E in [(3, 6144, 7), (5, 200, 4), (2, 128, 9)]:
        x = rng.integers(-3, 4, (n, H)).astype(np.float32)
        w = rng.integers(-3, 4, (E, H)).astype(np.float32)
        got = oracle.router_logits_bf16(bf16_bits(x), bf16_bits(w))
        assert np.array_equal(got, (x.astype(np.int64) @ w.T.astype(np.int64)).astype(np.float32))


def test_router_logits_bound_and_single_chunk(oracle):
    rng = np.random.default_rng(4)
    x = bf16_bits(rng.standard_normal((4, 6144)))
    w = bf16_bits(0.02 * rng.standard_normal((16, 6144)))
    got = oracle.router_logits_bf16(x, w).astype(np.float64)
    xf, wf = bits_to_f32(x).astype(np.float64), bits_to_f32(w).astype(np.float64)
    exact = xf @ wf.T
    bound = 6144 * np.finfo(np.float32).eps * (np.abs(xf) @ np.abs(wf).T)
    assert (np.abs(got - exact) <= bound).all()
    # One chunk (H <= 128) is exactly the reference linear_forward order.
    xs, ws = x[:, :128].copy(), w[:, :128].copy()
    assert np.array_equal(oracle.router_logits_bf16(xs, ws),
                          oracle.linear(bits_to_f32(xs), bits_to_f32(ws)))
    # ... and the chunked order differs from it in general (so the test above means something).
    assert not np.array_equal(oracle.router_logits_bf16(x, w), oracle.linear(xf.astype(np.float32),
                                                                              wf.astype(np.float32)))


def _brute_topk(oracle, logits, bias, k, norm, scale):
    n, E = logits.shape
    ids = np.zeros((n, k), np.int32)
    ws = np.zeros((n, k), np.float32)
    for t in range(n):
        sc = np.array([oracle.sigmoid(float(v)) for v in logits[t]], np.float32)
        ch = sc + (bias if bias is not None else np.float32(0))
        key = [(1 if np.isnan(c) else 0, -(c if not np.isnan(c) else 0), e) for e, c in enumerate(ch)]
        order = [e for _, _, e in sorted(key)][:k]
        ids[t] = order
        w = sc[order].astype(np.float32)
        s = np.float32(0)
        for v in w:
            s = np.float32(s + v)
        if norm and s > 0:
            w = (w / s).astype(np.float32)
        ws[t] = (w * np.float32(scale)).astype(np.float32)
    return ids, ws


@pytest.mark.parametrize("E,k,norm,scale", [(32, 4, True, 2.5), (256, 8, True, 2.5),
                                            (100, 8, False, 1.0), (8, 8, True, 2.5)])
def test_router_topk_vs_full_sort(oracle, E, k, norm, scale):
    rng = np.random.default_rng(E + k)
    logits = rng.standard_normal((40, E)).astype(np.float32)
    bias = rng.uniform(-0.1, 0.1, E).astype(np.float32)
    ids, w = oracle.router_topk(logits, bias, k, norm, scale)
    bid, bw = _brute_topk(oracle, logits, bias, k, norm, scale)
    assert np.array_equal(ids, bid)
    assert np.allclose(w, bw, rtol=0, atol=0)


def test_router_topk_ties_nan_bias(oracle):
    E, k = 16, 4
    logits = np.zeros((3, E), np.float32)
    logits[1, 5] = np.nan
    logits[2, :] = np.arange(E, dtype=np.float32)[::-1] * 0.01
    bias = np.zeros(E, np.float32)
    bias[9] = 1.0   # selection by choose, weight by the unbiased score
    ids, w = oracle.router_topk(logits, bias, k, True, 2.5)
    assert list(ids[0]) == [9, 0, 1, 2]              # ties -> lower index
    assert 5 not in ids[1]                           # NaN never beats a number
    assert ids[2][0] == 9 and list(ids[2][1:]) == [0, 1, 2]
    # weights are normalized unbiased scores x 2.5: all equal 0.5 in row 0
    assert np.allclose(w[0], 2.5 / 4)


# ---- dispatch -------------------------------------------------------------------

@pytest.mark.parametrize("n,k,E", [(1, 8, 256), (64, 8, 256), (37, 3, 5), (100, 4, 16)])
def test_dispatch_vs_stable_sort(oracle, n, k, E):
    rng = np.random.default_rng(n + E)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(n)]).astype(np.int32)
    off, st, sr = oracle.dispatch(ids, E)
    rows = sorted(((ids[t, s], t, s) for t in range(n) for s in range(k)))
    assert list(st) == [t for _, t, _ in rows] and list(sr) == [s for _, _, s in rows]
    counts = np.bincount(ids.ravel(), minlength=E)
    assert off[0] == 0 and off[E] == n * k and np.array_equal(np.diff(off), counts)
    # the inverse map round-trips
    pos = {(t, s): p for p, (t, s) in enumerate(zip(st, sr))}
    assert all(ids[t, s] == np.searchsorted(off, pos[(t, s)], side="right") - 1
               for t in range(n) for s in range(k))


# ---- whole layer ------------------------------------------------------------------

def _tiny_layer(seed, H=256, E=16, I=128, shared=True):
    rng = np.random.default_rng(seed)
    f = lambda *s: (0.02 * rng.standard_normal(s)).astype(np.float32)
    L = dict(rw=f(E, H), bias=rng.uniform(-0.1, 0.1, E).astype(np.float32),
             g=[f(I, H) for _ in range(E)], u=[f(I, H) for _ in range(E)],
             d=[f(H, I) for _ in range(E)])
    L["sh"] = (f(I, H), f(I, H), f(H, I)) if shared else None
    return L, rng


def test_moe_forward_vs_compiled_reference(oracle, ref):
    # hidden 256, 16 experts, top-4, I = S = 128, 64 tokens.
    L, rng = _tiny_layer(0)
    x = rng.standard_normal((64, 256)).astype(np.float32)
    out, ids, w = oracle.moe_forward(x, 16, 4, L["g"], L["u"], L["d"], L["sh"], router_w=L["rw"],
                                     e_bias=L["bias"], nthreads=4)
    rout, _ = ref.moe_mlp(x, L["rw"], L["bias"], L["g"], L["u"], L["d"], L["sh"], topk=4)
    # Only exp differs (std::exp vs the oracle's); any routing difference
    # would move outputs by O(0.1).
    assert np.max(np.abs(out - rout)) <= 1e-6 * max(1.0, np.max(np.abs(rout)))


@pytest.mark.parametrize("h_fp8", [False, True])
def test_moe_forward_streamed_equals_per_token(oracle, ref, h_fp8):
    # The expert-streamed form used for full-output GPU checks at large n
    # (row-batched expert FFN, then the slot-order combine) is the per-token
    # layer bit for bit: ragged expert groups (1 .. many rows, row blocks of
    # 32 with partial tails), empty experts, and the shared expert. Without
    # h quantization it also matches the compiled reference's moe_mlp.
    L, rng = _tiny_layer(3)
    n = 75
    x = rng.standard_normal((n, 256)).astype(np.float32)
    out, ids, w = oracle.moe_forward(x, 16, 4, L["g"], L["u"], L["d"], L["sh"], router_w=L["rw"],
                                     e_bias=L["bias"], nthreads=3, h_fp8=h_fp8)
    counts = np.bincount(ids.ravel(), minlength=16)
    assert counts.max() > 32 and counts.min() <= 16
    st = oracle.moe_forward_streamed(x, ids, w, lambda e: (L["g"][e], L["u"][e], L["d"][e]),
                                     L["sh"], h_fp8=h_fp8, nthreads=3)
    assert np.array_equal(st.view(np.uint32), out.view(np.uint32))
    if not h_fp8:
        rout, _ = ref.moe_mlp(x, L["rw"], L["bias"], L["g"], L["u"], L["d"], L["sh"], topk=4)
        assert np.max(np.abs(st - rout)) <= 1e-6 * max(1.0, np.max(np.abs(rout)))


def test_moe_forward_vs_fp64_bruteforce(oracle):
    L, rng = _tiny_layer(1)
    x = rng.standard_normal((8, 256)).astype(np.float32)
    out, ids, w = oracle.moe_forward(x, 16, 4, L["g"], L["u"], L["d"], L["sh"], router_w=L["rw"],
                                     e_bias=L["bias"])
    silu = lambda v: v / (1 + np.exp(-v))
    ffn = lambda g, u, d, xt: d.astype(np.float64) @ (silu(g.astype(np.float64) @ xt) * (u.astype(np.float64) @ xt))
    for t in range(8):
        xt = x[t].astype(np.float64)
        ref = sum(w[t, s] * ffn(L["g"][e], L["u"][e], L["d"][e], xt) for s, e in enumerate(ids[t]))
        ref = ref + ffn(*L["sh"], xt)
        assert np.max(np.abs(out[t] - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_moe_forward_special_cases(oracle):
    L, rng = _tiny_layer(2)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    # k = 1 with unit scale and normalization: weight 1 -> one plain SwiGLU MLP + shared.
    out, ids, w = oracle.moe_forward(x, 16, 1, L["g"], L["u"], L["d"], L["sh"], router_w=L["rw"],
                                     e_bias=L["bias"], routed_scale=1.0)
    assert np.all(w == 1.0)
    no_sh, _, _ = oracle.moe_forward(x, 16, 1, L["g"], L["u"], L["d"], None, router_w=L["rw"],
                                     e_bias=L["bias"], routed_scale=1.0)
    for t in range(4):
        e = ids[t, 0]
        h = np.array([oracle.silu(float(v)) for v in oracle.linear(x[t:t + 1], L["g"][e])[0]],
                     np.float32) * oracle.linear(x[t:t + 1], L["u"][e])[0]
        mlp = oracle.linear(h[None].astype(np.float32), L["d"][e])[0]
        assert np.allclose(no_sh[t], mlp, rtol=0, atol=1e-7)
    # Zero up-projections: every routed expert contributes exactly zero.
    zu = [np.zeros_like(u) for u in L["u"]]
    out_z, _, _ = oracle.moe_forward(x, 16, 4, L["g"], zu, L["d"], None, router_w=L["rw"],
                                     e_bias=L["bias"])
    assert np.all(out_z == 0.0)


# ---- FP8 activation quantization / block dequant ------------------------------

def test_quant_act_e4m3_vs_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(7)
    x = rng.standard_normal((6, 512)).astype(np.float32)
    x[2, 128:256] = 0.0                  # all-zero group -> scale 1, codes 0
    x[3, :128] *= 1e-6                   # tiny group
    q, s = oracle.quant_act_e4m3(x)
    g = np.abs(x.reshape(6, 4, 128)).max(axis=2)
    assert np.array_equal(s, np.where(g > 0, (g / np.float32(448.0)).astype(np.float32), 1.0))
    scaled = (x.reshape(6, 4, 128) / s[:, :, None]).astype(np.float32).reshape(6, 512)
    ref = torch.from_numpy(scaled).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(q, ref)
    assert np.all(q[2, 128:256] == 0)
    # each group's amax element maps to +-448 exactly
    for t in range(6):
        for gi in range(4):
            if g[t, gi] > 0:
                j = np.argmax(np.abs(x[t, gi * 128:(gi + 1) * 128]))
                assert q[t, gi * 128 + j] & 0x7F == 0x7E


def test_dequant_e4m3_blocks(oracle):
    rng = np.random.default_rng(8)
    q = rng.integers(0, 256, (256, 384), dtype=np.uint8)
    q[(q & 0x7F) == 0x7F] = 0x7E         # the encoder never emits the NaN codes
    s = rng.uniform(0.001, 0.01, (2, 3)).astype(np.float32)
    out = oracle.dequant_e4m3_blocks(q, s)
    for r, k in [(0, 0), (127, 127), (128, 0), (255, 383), (200, 130)]:
        assert out[r, k] == np.float32(oracle.e4m3_to_f32(int(q[r, k]))) * s[r // 128, k // 128]


def test_moe_forward_h_fp8(oracle):
    """FP8 layer intermediate: with k = 1, weight 1 and no shared expert the
    output is down . dequant(e4m3(h / s)) * s, h quantized per 128 features
    (the codes taken from torch's float8_e4m3fn conversion)."""
    torch = pytest.importorskip("torch")
    L, rng = _tiny_layer(3)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    plain, ids, w = oracle.moe_forward(x, 16, 1, L["g"], L["u"], L["d"], None, router_w=L["rw"],
                                       e_bias=L["bias"], routed_scale=1.0)
    q8, _, _ = oracle.moe_forward(x, 16, 1, L["g"], L["u"], L["d"], None, router_w=L["rw"],
                                  e_bias=L["bias"], routed_scale=1.0, h_fp8=True)
    for t in range(4):
        e = ids[t, 0]
        h = np.array([oracle.silu(float(v)) for v in oracle.linear(x[t:t + 1], L["g"][e])[0]],
                     np.float32) * oracle.linear(x[t:t + 1], L["u"][e])[0]
        s = (np.abs(h).max() / np.float32(448.0)).astype(np.float32)   # I = 128: one group
        codes = torch.from_numpy((h / s).astype(np.float32)).to(torch.float8_e4m3fn)
        hd = (codes.to(torch.float32).numpy() * s).astype(np.float32)
        ref = oracle.linear(hd[None], L["d"][e])[0]
        assert np.array_equal(q8[t], ref)
    # e4m3 keeps 3 mantissa bits: the layer moves by a few percent, not more.
    assert np.max(np.abs(q8 - plain)) <= 0.08 * np.max(np.abs(plain))


# ---- GGUF block formats ----------------------------------------------------

from moe_cases import GGUF_TYPES, random_gguf_rows  # noqa: E402


def test_gguf_tables_match_reference(oracle, ref):
    grid, iq4 = oracle.gguf_tables()
    rgrid, rsigns, riq4 = ref.gguf_tables()
    assert np.array_equal(grid, rgrid)
    assert np.array_equal(iq4, riq4)
    # the IQ2 sign table is the 7-bit index with an even-parity bit 7
    parity = np.array([i | ((bin(i).count("1") & 1) << 7) for i in range(128)], np.uint8)
    assert np.array_equal(parity, rsigns)


@pytest.mark.parametrize("qtype", sorted(GGUF_TYPES))
def test_gguf_dequant_bit_exact_vs_reference(oracle, ref, qtype):
    rng = np.random.default_rng(100 + qtype)
    n = 1024
    rows = random_gguf_rows(qtype, 6, n, rng)
    got = oracle.gguf_dequant_rows(qtype, rows, 6, n)
    for r in range(6):
        want = ref.gguf_dequant_row(qtype, rows[r], n)
        assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32)), r


def _f16(v):
    return np.array([v], np.float16).view(np.uint8)


def test_gguf_known_answers(oracle):
    # Q8_0: d = 1 -> the int8 codes themselves.
    b = np.zeros(34, np.uint8)
    b[0:2] = _f16(1.0)
    b[2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    assert np.array_equal(oracle.gguf_dequant_rows(8, b, 1, 32)[0], np.arange(-16, 16))
    # IQ4_XS: d = 1, every 6-bit scale 33 (lo 1, hi 2) -> scale 1, so element
    # values are the IQ4_NL table entries of their codes.
    _, iq4 = oracle.gguf_tables()
    b = np.zeros(136, np.uint8)
    b[0:2] = _f16(1.0)
    b[2:4] = np.array([0xAA, 0xAA], np.uint8)          # hi = 2 for all 8 sub-blocks
    b[4:8] = 0x11                                       # lo = 1 for all 8 sub-blocks
    codes = np.arange(256) % 16
    b[8:] = (codes[0::2][:128] | (codes[1::2][:128] << 4)).astype(np.uint8)
    y = oracle.gguf_dequant_rows(23, b, 1, 256)[0]
    for ib in range(8):
        q = b[8 + 16 * ib: 24 + 16 * ib]
        want = np.concatenate([iq4[q & 15], iq4[q >> 4]]).astype(np.float32)
        assert np.array_equal(y[32 * ib:32 * ib + 32], want)
    # Q6_K: d = 1, scales 1, ql / qh codes c -> c - 32.
    b = np.zeros(210, np.uint8)
    b[192:208] = 1
    b[208:210] = _f16(1.0)
    b[0:128] = 0x53        # low nibbles 3, high nibbles 5
    b[128:192] = 0b10010011   # 2-bit fields 3, 0, 1, 2
    y = oracle.gguf_dequant_rows(14, b, 1, 256)[0]
    assert np.all(y[0:32] == (3 | (3 << 4)) - 32)      # quarter 0: low nibble, bits 0-1
    assert np.all(y[32:64] == (3 | (0 << 4)) - 32)     # quarter 1: low nibble, bits 2-3
    assert np.all(y[64:96] == (5 | (1 << 4)) - 32)     # quarter 2: high nibble, bits 4-5
    assert np.all(y[96:128] == (5 | (2 << 4)) - 32)    # quarter 3: high nibble, bits 6-7
    # F16 / F32 rows are the values themselves.
    v = np.array([0.5, -2.0, 65504.0, 6.1e-5], np.float16)
    assert np.array_equal(oracle.gguf_dequant_rows(1, v.view(np.uint8), 1, 4)[0], v.astype(np.float32))


I8_TYPES = [8, 11, 12, 13, 14, 18, 23]


@pytest.mark.parametrize("qtype", I8_TYPES)
def test_gguf_int8_fragments_equal_the_decode(oracle, qtype):
    # weight = ds * wq - dm (the integer form the int8 path dots) reproduces the
    # block decode exactly, element by element.
    rng = np.random.default_rng(500 + qtype)
    n = 512
    rows = random_gguf_rows(qtype, 3, n, rng)
    W = oracle.gguf_dequant_rows(qtype, rows, 3, n)
    for r in range(3):
        for k in range(0, n, 8):
            wq, ds, dm = oracle.gguf_frag_i8(qtype, rows[r], k)
            w = np.float32(ds) * wq.astype(np.float32) - np.float32(dm)
            assert np.array_equal(w, W[r, k:k + 8]), (r, k)


def test_quant_act_q8_closed_form(oracle):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((5, 256)) * rng.uniform(0.01, 10, (5, 1))).astype(np.float32)
    x[2, 32:64] = 0.0                                  # an all-zero block
    q, s = oracle.quant_act_q8(x)
    xb = x.reshape(5, 8, 32)
    sx = (np.abs(xb).max(axis=2) / np.float32(127)).astype(np.float32)
    assert np.array_equal(s, sx)
    inv = np.where(sx > 0, np.float32(1) / np.where(sx > 0, sx, 1), 0).astype(np.float32)
    want = np.rint((xb * inv[:, :, None]).astype(np.float32)).astype(np.int8).reshape(5, 256)
    assert np.array_equal(q, want)
    assert np.all(q[2, 32:64] == 0) and s[2, 1] == 0
    err = np.abs(x.reshape(5, 8, 32) - s[:, :, None] * q.reshape(5, 8, 32).astype(np.float32))
    assert np.all(err <= s[:, :, None] * 0.5 * (1 + 1e-5))


def test_bf16_router_topk_agreement_with_fp32(oracle):
    # The fp32-activation entries round x and the router weights to bf16 and
    # then sum exact products in the fixed order; the reference's GPU router
    # is an fp32 GEMM (cuBLAS, TF32 by default: cuda/kernels.cuh:39-42). This
    # measures what that rounding costs in routing decisions on configs[1]-like
    # data (x N(0, 1), W N(0, 0.02), bias U(-0.1, 0.1), top-8 of 256): the
    # share of tokens whose top-8 set equals the one from exact logits (fp64
    # products of the fp32 inputs, rounded once), and the share of the
    # selected slots that agree. TF32 inputs (10-bit significands, the
    # reference's default) are measured beside it.
    def tf32(a):
        b = a.view(np.uint32).astype(np.uint64)
        return (((b + 0xFFF + ((b >> 13) & 1)) >> 13) << 13).astype(np.uint32).view(np.float32)

    sets_bf, slots_bf, sets_tf = [], [], []
    for seed in range(2):
        rng = np.random.default_rng(seed)
        n, H, E, k = 256, 6144, 256, 8
        x = rng.standard_normal((n, H)).astype(np.float32)
        W = (0.02 * rng.standard_normal((E, H))).astype(np.float32)
        eb = rng.uniform(-0.1, 0.1, E).astype(np.float32)
        exact = (x.astype(np.float64) @ W.astype(np.float64).T).astype(np.float32)
        tf = (tf32(x).astype(np.float64) @ tf32(W).astype(np.float64).T).astype(np.float32)
        bf = oracle.router_logits_bf16(bf16_bits(x), bf16_bits(W))
        ie, _ = oracle.router_topk(exact, eb, k, True, 2.5)
        ib, _ = oracle.router_topk(bf, eb, k, True, 2.5)
        it, _ = oracle.router_topk(tf, eb, k, True, 2.5)
        sets_bf += [set(a) == set(b) for a, b in zip(ib, ie)]
        slots_bf += [len(set(a) & set(b)) / k for a, b in zip(ib, ie)]
        sets_tf += [set(a) == set(b) for a, b in zip(it, ie)]
    # Measured: bf16 0.98 of the tokens (0.998 of the slots), TF32 0.998.
    assert np.mean(sets_bf) >= 0.95 and np.mean(slots_bf) >= 0.99
    assert np.mean(sets_tf) >= np.mean(sets_bf)
