"""Minimal GGUF v3 writer for test models (numpy only).

Layout written: header (magic, version 3, tensor count, KV count), KV pairs,
tensor infos (name, dims in GGUF order ne[0]=columns first, ggml type, offset
relative to the data section), zero padding to a 32-byte boundary, then the
tensor data, each tensor starting on a 32-byte boundary.  The KV keys are
written in the order the reference loader's substring scan needs
(`head_count` before `head_count_kv`, `vocab_size` present) -- the same order
as the reference's own synthetic-model writer (tests/test_e2e.c:105-115).
"""
import struct
import numpy as np

from _native import Q4_BLOCK, Q8_BLOCK

GGUF_MAGIC = 0x46554747
T_U32, T_F32, T_STR = 4, 6, 8
GGML_F32, GGML_Q4_0, GGML_Q8_0 = 0, 2, 8


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def write_gguf(path, kv, tensors, alignment=32):
    """kv: list of (key, type, value); tensors: list of (name, ggml_type, dims, bytes)."""
    out = bytearray()
    out += struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(kv))
    for key, t, v in kv:
        out += _str(key) + struct.pack("<I", t)
        if t == T_U32:
            out += struct.pack("<I", v)
        elif t == T_F32:
            out += struct.pack("<f", v)
        elif t == T_STR:
            out += _str(v)
        else:
            raise ValueError(t)
    offsets = []
    off = 0
    for name, gt, dims, data in tensors:
        offsets.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, gt, dims, data), o in zip(tensors, offsets):
        out += _str(name) + struct.pack("<I", len(dims))
        for dmn in dims:
            out += struct.pack("<Q", dmn)
        out += struct.pack("<IQ", gt, o)
    pad = (-len(out)) % alignment
    out += b"\0" * pad
    base = len(out)
    for (name, gt, dims, data), o in zip(tensors, offsets):
        cur = len(out) - base
        out += b"\0" * (o - cur)
        out += data
    out += b"\0" * ((-len(out)) % alignment)
    with open(path, "wb") as f:
        f.write(out)


def quantize_q4_0_np(x):
    """Vectorised restatement of the reference Q4_0 writer (src/quantize.c:88-114)
    for rows whose length is a multiple of 32: d = amax/7 (>=1e-10), stored as
    truncated fp16, q = trunc(x * (1/d)) clamped to [-8, 7] + 8."""
    x = np.asarray(x, dtype=np.float32)
    rows, cols = x.shape
    xb = x.reshape(rows, cols // 32, 32)
    amax = np.max(np.abs(xb), axis=2)
    d = (amax / np.float32(7.0)).astype(np.float32)
    d = np.where(d < np.float32(1e-10), np.float32(1e-10), d).astype(np.float32)
    inv = (np.float32(1.0) / d).astype(np.float32)
    q = np.trunc((xb * inv[..., None]).astype(np.float32)).astype(np.int64)
    q = np.clip(q, -8, 7) + 8
    blocks = np.zeros((rows, cols // 32), dtype=Q4_BLOCK)
    blocks["d"] = fp32_to_fp16_trunc(d)
    blocks["qs"] = (q[..., 0::2] | (q[..., 1::2] << 4)).astype(np.uint8)
    return blocks


def fp32_to_fp16_trunc(f):
    """Truncating, flush-to-zero conversion (src/quantize.c:17-35)."""
    b = np.asarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    sign = ((b >> 31) << 15).astype(np.uint64)
    e = (b >> 23) & 0xFF
    m = b & 0x7FFFFF
    he = e.astype(np.int64) - 112
    out = np.where(he <= 0, sign, sign | (np.clip(he, 0, 31).astype(np.uint64) << 10) | (m >> 13))
    out = np.where(he >= 31, sign | 0x7C00, out)
    out = np.where(e == 0, sign, out)
    out = np.where(e == 0xFF, sign | 0x7C00 | (m >> 13), out)
    return out.astype(np.uint16)


def llama_gguf(path, rng, n_layers, n_embd, n_heads, n_kv_heads, n_ff, n_vocab,
               rope_theta=10000.0, std=0.02, with_attn_output=True, norm_random=False,
               emb_type=GGML_Q4_0, out_type=GGML_Q4_0, with_output=True, matrix_type=GGML_Q4_0):
    """Write a random-init Llama-style model (weights N(0, std) quantised with
    the reference quantiser or kept F32, norms F32).  Returns dict of the raw
    arrays."""
    hd = n_embd // n_heads
    kvd = n_kv_heads * hd
    kv = [
        ("general.architecture", T_STR, "llama"),
        ("llama.block_count", T_U32, n_layers),
        ("llama.attention.head_count", T_U32, n_heads),
        ("llama.attention.head_count_kv", T_U32, n_kv_heads),
        ("llama.embedding_length", T_U32, n_embd),
        ("llama.feedforward_length", T_U32, n_ff),
        ("llama.rope.freq_base", T_F32, rope_theta),
        ("llama.vocab_size", T_U32, n_vocab),
    ]
    tensors = []
    raw = {}

    def qmat(name, rows, cols, gt=GGML_Q4_0):
        w = rng.normal(0.0, std, size=(rows, cols)).astype(np.float32)
        if gt == GGML_F32:
            b = w
        elif gt == GGML_Q4_0:
            b = quantize_q4_0_np(w)
        else:
            b = quantize_q8_0_np(w)
        raw[name] = b
        tensors.append((name, gt, [cols, rows], b.tobytes()))

    def norm(name, n):
        w = (rng.uniform(0.5, 1.5, size=n) if norm_random else np.ones(n)).astype(np.float32)
        raw[name] = w
        tensors.append((name, GGML_F32, [n], w.tobytes()))

    qmat("token_embd.weight", n_vocab, n_embd, emb_type)
    for l in range(n_layers):
        norm(f"blk.{l}.attn_norm.weight", n_embd)
        qmat(f"blk.{l}.attn_q.weight", n_embd, n_embd, matrix_type)
        qmat(f"blk.{l}.attn_k.weight", kvd, n_embd, matrix_type)
        qmat(f"blk.{l}.attn_v.weight", kvd, n_embd, matrix_type)
        if with_attn_output:
            qmat(f"blk.{l}.attn_output.weight", n_embd, n_embd, matrix_type)
        norm(f"blk.{l}.ffn_norm.weight", n_embd)
        qmat(f"blk.{l}.ffn_gate.weight", n_ff, n_embd, matrix_type)
        qmat(f"blk.{l}.ffn_up.weight", n_ff, n_embd, matrix_type)
        qmat(f"blk.{l}.ffn_down.weight", n_embd, n_ff, matrix_type)
    norm("output_norm.weight", n_embd)
    if with_output:
        qmat("output.weight", n_vocab, n_embd, out_type)
    write_gguf(path, kv, tensors)
    return raw


def quantize_q8_0_np(x):
    """Build-defined Q8_0 writer (the reference has none): d = amax/127 stored
    as round-to-nearest fp16, q = round-half-away(x / d) clamped to [-127, 127]."""
    x = np.asarray(x, dtype=np.float32)
    rows, cols = x.shape
    xb = x.reshape(rows, cols // 32, 32)
    amax = np.max(np.abs(xb), axis=2)
    d = (amax / np.float32(127.0)).astype(np.float32)
    dh = d.astype(np.float16)
    dq = dh.astype(np.float32)
    inv = np.where(dq > 0, np.float32(1.0) / np.where(dq > 0, dq, 1), 0).astype(np.float32)
    q = np.sign(xb) * np.floor(np.abs(xb * inv[..., None]) + 0.5)
    q = np.clip(q, -127, 127).astype(np.int8)
    blocks = np.zeros((rows, cols // 32), dtype=Q8_BLOCK)
    blocks["d"] = dh.view(np.uint16)
    blocks["qs"] = q
    return blocks
