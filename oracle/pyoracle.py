"""ctypes bindings for the CPU checker libraries (test infrastructure only)."""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "libmoe_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libglmref.so")
REF_TREE = "/root/reference"

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64 = C.c_int64


def build(with_ref=None):
    """Compile the oracle (always) and oracle/_ref (when the reference tree exists)."""
    subprocess.run(["make", "-s", "-C", HERE, "oracle"], check=True)
    if with_ref is None:
        with_ref = os.path.isdir(os.path.join(REF_TREE, "src"))
    if with_ref:
        subprocess.run(["make", "-s", "-j8", "-C", HERE, "ref", f"REF={REF_TREE}"], check=True)


def _ptr_array(arrs):
    """Array of float* (NULL for None) for the per-expert weight lists."""
    out = (C.c_void_p * len(arrs))()
    for i, a in enumerate(arrs):
        out[i] = None if a is None else a.ctypes.data
    return out


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            build(with_ref=False)
        L = C.CDLL(path)
        self.L = L
        L.orc_expf.restype = C.c_float
        L.orc_expf.argtypes = [C.c_float]
        L.orc_sigmoid.restype = C.c_float
        L.orc_sigmoid.argtypes = [C.c_float]
        L.orc_silu.restype = C.c_float
        L.orc_silu.argtypes = [C.c_float]
        L.orc_f32_to_bf16_n.argtypes = [_f32p, _u16p, _i64]
        L.orc_bf16_to_f32_n.argtypes = [_u16p, _f32p, _i64]
        L.orc_e4m3_to_f32.restype = C.c_float
        L.orc_e4m3_to_f32.argtypes = [C.c_uint8]
        L.orc_f32_to_e4m3.restype = C.c_uint8
        L.orc_f32_to_e4m3.argtypes = [C.c_float]
        L.orc_quant_act_e4m3.argtypes = [_f32p, _i64, _i64, _u8p, _f32p]
        L.orc_dequant_e4m3_blocks.argtypes = [_u8p, _f32p, _i64, _i64, _f32p]
        L.orc_linear_f32.argtypes = [_f32p, _f32p, _i64, _i64, _i64, _f32p]
        L.orc_router_logits_bf16.argtypes = [_u16p, _u16p, _i64, _i64, _i64, _f32p]
        L.orc_router_topk.argtypes = [_f32p, C.c_void_p, _i64, C.c_int, C.c_int, C.c_int,
                                      C.c_float, _i32p, _f32p]
        L.orc_dispatch.argtypes = [_i32p, _i64, C.c_int, C.c_int, _i32p, _i32p, _i32p]
        L.orc_dequant_int4_rows.argtypes = [_u8p, _f32p, _i64, _i64, _i64, _f32p]
        L.orc_quantize_w4_rows.argtypes = [_f32p, _i64, _i64, _i64, _u8p, _f32p]
        L.orc_moe_forward.argtypes = [
            _f32p, _i64, _i64, C.c_int, C.c_int, _i64, _i64, C.c_void_p, C.c_void_p,
            C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
            C.c_void_p, C.c_int, C.c_float, C.c_int, _f32p, _i32p, _f32p]
        L.orc_moe_forward_ex.argtypes = [
            _f32p, _i64, _i64, C.c_int, C.c_int, _i64, _i64, C.c_void_p, C.c_void_p,
            C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
            C.c_void_p, C.c_int, C.c_float, C.c_int, C.c_int, _f32p, _i32p, _f32p]
        L.orc_expert_rows.argtypes = [_f32p, _i64, _i64, _i64, _f32p, _f32p, _f32p, C.c_int,
                                      C.c_int, _f32p]
        L.orc_combine_slots.argtypes = [_f32p, _f32p, C.c_void_p, _i64, C.c_int, _i64, _f32p]
        L.orc_gguf_block_elems.restype = _i64
        L.orc_gguf_block_elems.argtypes = [C.c_uint32]
        L.orc_gguf_block_bytes.restype = _i64
        L.orc_gguf_block_bytes.argtypes = [C.c_uint32]
        L.orc_gguf_value.restype = C.c_float
        L.orc_gguf_value.argtypes = [C.c_uint32, _u8p, C.c_int]
        L.orc_gguf_dequant_row.restype = C.c_int
        L.orc_gguf_dequant_row.argtypes = [C.c_uint32, _u8p, _i64, _f32p]
        L.orc_gguf_tables.argtypes = [C.POINTER(C.POINTER(C.c_uint32)),
                                      C.POINTER(C.POINTER(C.c_int8))]
        _i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
        _f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
        L.orc_quant_act_q8.argtypes = [_f32p, _i64, _i64, _i8p, _f32p]
        L.orc_gguf_frag_i8.restype = C.c_int
        L.orc_gguf_frag_i8.argtypes = [C.c_uint32, _u8p, _i64, _i8p, C.POINTER(C.c_float),
                                       C.POINTER(C.c_float)]
        L.orc_gemm_q_i8.restype = C.c_int
        L.orc_gemm_q_i8.argtypes = [C.c_uint32, _i8p, _f32p, _u8p, _i64, _i64, _i64, _i64, _f64p]

    # scalar helpers
    def expf(self, x):
        return self.L.orc_expf(x)

    def sigmoid(self, x):
        return self.L.orc_sigmoid(x)

    def silu(self, x):
        return self.L.orc_silu(x)

    def f32_to_bf16(self, a):
        a = np.ascontiguousarray(a, np.float32)
        out = np.empty(a.shape, np.uint16)
        self.L.orc_f32_to_bf16_n(a.ravel(), out.ravel(), a.size)
        return out

    def bf16_to_f32(self, a):
        a = np.ascontiguousarray(a, np.uint16)
        out = np.empty(a.shape, np.float32)
        self.L.orc_bf16_to_f32_n(a.ravel(), out.ravel(), a.size)
        return out

    def e4m3_to_f32(self, v):
        return self.L.orc_e4m3_to_f32(int(v))

    def f32_to_e4m3(self, f):
        return self.L.orc_f32_to_e4m3(float(f))

    def quant_act_e4m3(self, x):
        x = np.ascontiguousarray(x, np.float32)
        n, K = x.shape
        q = np.empty((n, K), np.uint8)
        s = np.empty((n, K // 128), np.float32)
        self.L.orc_quant_act_e4m3(x, n, K, q, s)
        return q, s

    def dequant_e4m3_blocks(self, q, scales):
        q = np.ascontiguousarray(q, np.uint8)
        rows, K = q.shape
        out = np.empty((rows, K), np.float32)
        self.L.orc_dequant_e4m3_blocks(q, np.ascontiguousarray(scales, np.float32), rows, K, out)
        return out

    def linear(self, x, w):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        n, i = x.shape
        o = w.shape[0]
        y = np.empty((n, o), np.float32)
        self.L.orc_linear_f32(x, w, n, i, o, y)
        return y

    def router_logits_bf16(self, x_bf16, wr_bf16):
        x = np.ascontiguousarray(x_bf16, np.uint16)
        w = np.ascontiguousarray(wr_bf16, np.uint16)
        n, H = x.shape
        E = w.shape[0]
        y = np.empty((n, E), np.float32)
        self.L.orc_router_logits_bf16(x, w, n, H, E, y)
        return y

    def router_topk(self, logits, e_bias, topk, norm_topk=True, routed_scale=2.5):
        lg = np.ascontiguousarray(logits, np.float32)
        n, E = lg.shape
        ids = np.empty((n, topk), np.int32)
        w = np.empty((n, topk), np.float32)
        b = None if e_bias is None else np.ascontiguousarray(e_bias, np.float32)
        rc = self.L.orc_router_topk(lg, None if b is None else b.ctypes.data, n, E, topk,
                                    int(norm_topk), routed_scale, ids, w)
        if rc:
            raise ValueError("orc_router_topk: bad shape")
        return ids, w

    def dispatch(self, ids, E):
        ids = np.ascontiguousarray(ids, np.int32)
        n, k = ids.shape
        off = np.empty(E + 1, np.int32)
        st = np.empty(n * k, np.int32)
        sr = np.empty(n * k, np.int32)
        if self.L.orc_dispatch(ids, n, k, E, off, st, sr):
            raise ValueError("orc_dispatch: expert id out of range")
        return off, st, sr

    def gguf_block(self, qtype):
        """(elements, bytes) of one block of a GGUF type (0, 0 if unsupported)."""
        return self.L.orc_gguf_block_elems(qtype), self.L.orc_gguf_block_bytes(qtype)

    def gguf_dequant_rows(self, qtype, data, rows, n):
        """rows x n fp32 from GGUF rows stored back to back (uint8 array)."""
        be, bb = self.gguf_block(qtype)
        rb = n // be * bb
        data = np.ascontiguousarray(data, np.uint8).reshape(-1)
        out = np.empty((rows, n), np.float32)
        for r in range(rows):
            if self.L.orc_gguf_dequant_row(qtype, data[r * rb:(r + 1) * rb], n, out[r]):
                raise ValueError(f"orc_gguf_dequant_row: type {qtype}")
        return out

    def quant_act_q8(self, x):
        """x [n, in] fp32 -> (xq [n, in] int8, xs [n, in/32] fp32)."""
        x = np.ascontiguousarray(x, np.float32)
        n, i = x.shape
        q = np.empty((n, i), np.int8)
        s = np.empty((n, i // 32), np.float32)
        self.L.orc_quant_act_q8(x, n, i, q, s)
        return q, s

    def gguf_frag_i8(self, qtype, row, k):
        wq = np.empty(8, np.int8)
        ds, dm = C.c_float(), C.c_float()
        if self.L.orc_gguf_frag_i8(qtype, np.ascontiguousarray(row, np.uint8), k, wq,
                                   C.byref(ds), C.byref(dm)):
            raise ValueError(f"orc_gguf_frag_i8: type {qtype}")
        return wq, ds.value, dm.value

    def gemm_q_i8(self, qtype, xq, xs, w, out, row_bytes):
        """gemm_q_i8's sums in fp64: y [n, out]."""
        xq = np.ascontiguousarray(xq, np.int8)
        n, i = xq.shape
        y = np.empty((n, out), np.float64)
        if self.L.orc_gemm_q_i8(qtype, xq, np.ascontiguousarray(xs, np.float32),
                                np.ascontiguousarray(w, np.uint8).reshape(-1), n, i, out,
                                row_bytes, y):
            raise ValueError(f"orc_gemm_q_i8: type {qtype}")
        return y

    def gguf_tables(self):
        g = C.POINTER(C.c_uint32)()
        k = C.POINTER(C.c_int8)()
        self.L.orc_gguf_tables(C.byref(g), C.byref(k))
        return (np.ctypeslib.as_array(g, (256,)).copy(), np.ctypeslib.as_array(k, (16,)).copy())

    def dequant_int4_rows(self, q, scales, in_features, group_size):
        q = np.ascontiguousarray(q, np.uint8)
        s = np.ascontiguousarray(scales, np.float32)
        rows = q.shape[0]
        out = np.empty((rows, in_features), np.float32)
        self.L.orc_dequant_int4_rows(q, s, rows, in_features, group_size, out)
        return out

    def quantize_w4_rows(self, w, group_size):
        w = np.ascontiguousarray(w, np.float32)
        rows, i = w.shape
        q = np.empty((rows, (i + 1) // 2), np.uint8)
        s = np.empty((rows, (i + group_size - 1) // group_size), np.float32)
        self.L.orc_quantize_w4_rows(w, rows, i, group_size, q, s)
        return q, s

    def expert_rows(self, x, gate, up, down, h_fp8=False, nthreads=1, out=None):
        """One expert's FFN on the rows of x [m, H] (orc_ffn per row, bit for bit)."""
        x = np.ascontiguousarray(x, np.float32)
        m, H = x.shape
        I = gate.shape[0]
        y = np.empty((m, H), np.float32) if out is None else out
        assert y.shape == (m, H) and y.dtype == np.float32 and y.flags.c_contiguous
        self.L.orc_expert_rows(x, m, H, I, np.ascontiguousarray(gate, np.float32),
                               np.ascontiguousarray(up, np.float32),
                               np.ascontiguousarray(down, np.float32), int(h_fp8), nthreads, y)
        return y

    def combine_slots(self, slot_rows, topk_w, shared_rows=None):
        """out[t] = ((0 + w0*y0) + w1*y1 + ...) + y_shared[t] (orc_moe_worker's order)."""
        slot_rows = np.ascontiguousarray(slot_rows, np.float32)
        topk_w = np.ascontiguousarray(topk_w, np.float32)
        n, topk = topk_w.shape
        H = slot_rows.shape[-1]
        assert slot_rows.size == n * topk * H
        sh = None
        if shared_rows is not None:
            sh = np.ascontiguousarray(shared_rows, np.float32)
            assert sh.shape == (n, H)
        out = np.empty((n, H), np.float32)
        self.L.orc_combine_slots(slot_rows, topk_w, None if sh is None else sh.ctypes.data, n,
                                 topk, H, out)
        return out

    def moe_forward_streamed(self, x, ids, w, expert, shared=None, h_fp8=False, nthreads=8):
        """The layer for given routing (ids, w [n, topk]) with the experts
        materialized one at a time: expert(e) -> (gate, up, down) fp32. Equals
        moe_forward on the same routing bit for bit, at a fraction of the memory
        (one expert's weights at a time) and with row-batched arithmetic."""
        x = np.ascontiguousarray(x, np.float32)
        n, H = x.shape
        ids = np.asarray(ids)
        topk = ids.shape[1]
        slots = np.empty((n * topk, H), np.float32)
        flat = ids.ravel()
        order = np.argsort(flat, kind="stable")
        bounds = np.searchsorted(flat[order], np.arange(flat.max() + 2 if n else 1))
        for e in np.unique(flat):
            rows = order[bounds[e]:bounds[e + 1]]
            g, u, d = expert(int(e))
            slots[rows] = self.expert_rows(x[rows // topk], g, u, d, h_fp8, nthreads)
        sh_rows = None
        if shared is not None:
            g, u, d = shared
            sh_rows = self.expert_rows(x, g, u, d, h_fp8, nthreads)
        return self.combine_slots(slots, w, sh_rows)

    def moe_forward(self, x, E, topk, gate, up, down, sh=None, router_w=None, logits=None,
                    e_bias=None, norm_topk=True, routed_scale=2.5, nthreads=1, h_fp8=False):
        """gate/up/down: lists of E fp32 arrays (or None for an unmaterialized expert).
        h_fp8: quantize the intermediate h per 128 features to e4m3 (FP8 layer)."""
        x = np.ascontiguousarray(x, np.float32)
        n, H = x.shape
        I = next(g for g in gate if g is not None).shape[0]
        S = sh[0].shape[0] if sh is not None else 0
        keep = [np.ascontiguousarray(a, np.float32) if a is not None else None
                for a in list(gate) + list(up) + list(down)]
        g_, u_, d_ = keep[:E], keep[E:2 * E], keep[2 * E:]
        shk = [np.ascontiguousarray(a, np.float32) for a in sh] if sh is not None else None
        rw = None if router_w is None else np.ascontiguousarray(router_w, np.float32)
        lg = None if logits is None else np.ascontiguousarray(logits, np.float32)
        eb = None if e_bias is None else np.ascontiguousarray(e_bias, np.float32)
        out = np.empty((n, H), np.float32)
        ids = np.empty((n, topk), np.int32)
        w = np.empty((n, topk), np.float32)
        rc = self.L.orc_moe_forward_ex(
            x, n, H, E, topk, I, S, None if rw is None else rw.ctypes.data,
            None if lg is None else lg.ctypes.data, None if eb is None else eb.ctypes.data,
            _ptr_array(g_), _ptr_array(u_), _ptr_array(d_),
            None if shk is None else shk[0].ctypes.data,
            None if shk is None else shk[1].ctypes.data,
            None if shk is None else shk[2].ctypes.data,
            int(norm_topk), routed_scale, int(h_fp8), nthreads, out, ids, w)
        if rc:
            raise ValueError("orc_moe_forward: routing selected an unmaterialized expert")
        return out, ids, w


class RefLib:
    """glmserve's compiled CPU MoE path (oracle/_ref/libglmref.so)."""

    def __init__(self, path=REF_SO):
        L = C.CDLL(path)
        self.L = L
        L.ref_hw_threads.restype = C.c_int
        L.ref_hardware_concurrency.restype = C.c_int
        L.ref_dequant_int4.argtypes = [_u8p, _f32p, _i64, _i64, _f32p]
        L.ref_moe_mlp.restype = C.c_int
        L.ref_gguf_dequant_row.restype = C.c_int
        L.ref_gguf_dequant_row.argtypes = [C.c_uint32, _u8p, _i64, _f32p]
        L.ref_gguf_tables.argtypes = [C.POINTER(C.POINTER(C.c_uint8)),
                                      C.POINTER(C.POINTER(C.c_uint8)),
                                      C.POINTER(C.POINTER(C.c_int8))]
        L.ref_moe_mlp.argtypes = [
            _f32p, _i64, _i64, C.c_int, C.c_int, _i64, _i64, _f32p, C.c_void_p,
            C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
            C.c_int, C.c_double, _f32p, C.POINTER(C.c_double)]

    def hw_threads(self):
        return self.L.ref_hw_threads()

    def gguf_dequant_row(self, qtype, data, n):
        out = np.empty(n, np.float32)
        if self.L.ref_gguf_dequant_row(qtype, np.ascontiguousarray(data, np.uint8), n, out):
            raise ValueError(f"ref_gguf_dequant_row: type {qtype}")
        return out

    def gguf_tables(self):
        g = C.POINTER(C.c_uint8)()
        s = C.POINTER(C.c_uint8)()
        k = C.POINTER(C.c_int8)()
        self.L.ref_gguf_tables(C.byref(g), C.byref(s), C.byref(k))
        return (np.ctypeslib.as_array(g, (1024,)).copy().view(np.uint32),
                np.ctypeslib.as_array(s, (128,)).copy(), np.ctypeslib.as_array(k, (16,)).copy())

    def hardware_concurrency(self):
        return self.L.ref_hardware_concurrency()

    def dequant_int4(self, packed, scales, count, group_size):
        out = np.empty(count, np.float32)
        self.L.ref_dequant_int4(np.ascontiguousarray(packed, np.uint8),
                                np.ascontiguousarray(scales, np.float32), count, group_size, out)
        return out

    def moe_mlp(self, x, router_w, e_bias, gate, up, down, sh=None, topk=8, norm_topk=True,
                routed_scale=2.5):
        """Returns (out, seconds_of_the_moe_mlp_call)."""
        x = np.ascontiguousarray(x, np.float32)
        n, H = x.shape
        E = router_w.shape[0]
        I = next(g for g in gate if g is not None).shape[0]
        S = sh[0].shape[0] if sh is not None else 0
        keep = [np.ascontiguousarray(a, np.float32) if a is not None else None
                for a in list(gate) + list(up) + list(down)]
        shk = [np.ascontiguousarray(a, np.float32) for a in sh] if sh is not None else None
        eb = None if e_bias is None else np.ascontiguousarray(e_bias, np.float32)
        out = np.empty((n, H), np.float32)
        secs = C.c_double(0.0)
        rc = self.L.ref_moe_mlp(
            x, n, H, E, topk, I, S, np.ascontiguousarray(router_w, np.float32),
            None if eb is None else eb.ctypes.data,
            _ptr_array(keep[:E]), _ptr_array(keep[E:2 * E]), _ptr_array(keep[2 * E:]),
            None if shk is None else shk[0].ctypes.data,
            None if shk is None else shk[1].ctypes.data,
            None if shk is None else shk[2].ctypes.data,
            int(norm_topk), float(routed_scale), out, C.byref(secs))
        if rc:
            raise RuntimeError("reference moe_mlp raised")
        return out, secs.value


_ORACLE = None


def load_oracle():
    global _ORACLE
    if _ORACLE is None:
        _ORACLE = Oracle()
    return _ORACLE


def load_ref():
    """The compiled reference, or None when oracle/_ref was not built."""
    if not os.path.exists(REF_SO):
        return None
    return RefLib()
