"""Build an oracle or_model (oracle/oracle.h) from numpy arrays."""
import ctypes as C
import numpy as np

from _native import OrMat, OrModel

TYPE_CODE = {"f32": 0, "q4_0": 2, "q8_0": 8}


def _mat(arr, rows, cols):
    m = OrMat()
    if arr is None:
        m.type, m.data, m.rows, m.cols = 0, None, rows, cols
        return m
    if arr.dtype.names:  # block array
        m.type = 2 if arr.dtype.itemsize == 18 else 8
    else:
        m.type = 0
    m.data = arr.ctypes.data_as(C.c_void_p)
    m.rows, m.cols = rows, cols
    return m


class OracleModel:
    """Holds numpy buffers alive and exposes an OrModel pointer.

    weights: dict name -> array, GGUF names (token_embd.weight, blk.L.attn_q.weight,
    ..., output_norm.weight, output.weight).  Block arrays are (rows, cols/32).
    """

    def __init__(self, weights, n_layers, n_embd, n_heads, n_kv_heads, n_ff, n_vocab, n_ctx,
                 rope_theta=10000.0, q4_mode=0, attn_cap=4096, attn_o_inplace=0, gate_thr=0.01,
                 wscale=1.0, kv_half=0):
        self.keep = []
        hd = n_embd // n_heads
        kvd = n_kv_heads * hd
        m = OrModel()
        m.n_layers, m.n_heads, m.n_kv_heads, m.n_embd = n_layers, n_heads, n_kv_heads, n_embd
        m.n_head_dim, m.n_ff, m.n_vocab, m.n_ctx = hd, n_ff, n_vocab, n_ctx
        m.rope_theta, m.q4_mode, m.attn_cap, m.attn_o_inplace = rope_theta, q4_mode, attn_cap, attn_o_inplace
        m.gate_thr, m.wscale = gate_thr, wscale
        m.kv_half = kv_half

        def W(name):
            a = weights.get(name)
            if a is not None:
                a = np.ascontiguousarray(a)
                self.keep.append(a)
            return a

        emb = W("token_embd.weight")
        m.tok_embd = _mat(emb, n_vocab, n_embd)
        out = W("output.weight")
        if out is None:
            out = emb  # output falls back to tok_embd (src/format.c:237-238)
        m.output = _mat(out, n_vocab, n_embd)
        on = W("output_norm.weight")
        m.has_out_norm = 1 if "output_norm.weight" in weights else 0
        m.out_norm = on.ctypes.data_as(C.c_void_p) if (on is not None and on.dtype == np.float32) else None

        def mats(suffix, rows, cols):
            arr = (OrMat * n_layers)()
            for l in range(n_layers):
                arr[l] = _mat(W(f"blk.{l}.{suffix}"), rows, cols)
            self.keep.append(arr)
            return C.cast(arr, C.c_void_p)

        m.wq = mats("attn_q.weight", n_embd, n_embd)
        m.wk = mats("attn_k.weight", kvd, n_embd)
        m.wv = mats("attn_v.weight", kvd, n_embd)
        m.wo = mats("attn_output.weight", n_embd, n_embd)
        m.wg = mats("ffn_gate.weight", n_ff, n_embd)
        m.wu = mats("ffn_up.weight", n_ff, n_embd)
        m.wd = mats("ffn_down.weight", n_embd, n_ff)

        def vecs(suffix):
            arr = (C.c_void_p * n_layers)()
            for l in range(n_layers):
                a = W(f"blk.{l}.{suffix}")
                arr[l] = a.ctypes.data if (a is not None and a.dtype == np.float32) else None
            self.keep.append(arr)
            return C.cast(arr, C.c_void_p)

        m.attn_norm = vecs("attn_norm.weight")
        m.ffn_norm = vecs("ffn_norm.weight")
        m.bq = vecs("attn_q.bias")
        m.bk = vecs("attn_k.bias")
        m.bv = vecs("attn_v.bias")
        self.k_cache = np.zeros(n_layers * n_ctx * kvd, dtype=np.float32)
        self.v_cache = np.zeros(n_layers * n_ctx * kvd, dtype=np.float32)
        m.k_cache = self.k_cache.ctypes.data_as(C.c_void_p)
        m.v_cache = self.v_cache.ctypes.data_as(C.c_void_p)
        m.cache_len = 0
        self.m = m
        self.n_vocab = n_vocab

    @property
    def ptr(self):
        return C.byref(self.m)

    @property
    def cache_len(self):
        return self.m.cache_len

    @cache_len.setter
    def cache_len(self, v):
        self.m.cache_len = v
