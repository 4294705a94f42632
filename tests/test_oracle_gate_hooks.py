"""Pins of the oracle's FFN gate-skip test hooks (CPU only).

The hooks (or_model.gate_near / gate_near_idx / flip) let a GPU parity test
prove that a logit difference comes from one skip decision at the threshold
|silu(g_i)| < thr (src/model.c:582-585): the log names the column closest to
the threshold, and the flip reruns the oracle with exactly that decision
inverted.  The checks below tie both hooks to independent computations:

* flip of a computed column == the same model with that up row's weights
  zeroed (bit-exact), and two flips == two zeroed rows;
* flip of a skipped column == a model with no skipping whose other up rows
  are zeroed (bit-exact);
* the logged column and distance == numpy float64 of the first layer's gate.
"""
import ctypes as C

import numpy as np

import _native as N
from _gguf import llama_gguf
from _oracle_model import OracleModel

O = N.oracle()
SHAPE = dict(n_layers=1, n_embd=64, n_heads=4, n_kv_heads=2, n_ff=96, n_vocab=40)


def model(tmp_path, seed=3):
    rng = np.random.default_rng(seed)
    s = SHAPE
    raw = llama_gguf(str(tmp_path / "m.gguf"), rng, s["n_layers"], s["n_embd"], s["n_heads"],
                     s["n_kv_heads"], s["n_ff"], s["n_vocab"], std=0.08)
    return raw


def run(raw, tok, thr, flip=None, log=False):
    s = SHAPE
    om = OracleModel(raw, s["n_layers"], s["n_embd"], s["n_heads"], s["n_kv_heads"], s["n_ff"],
                     s["n_vocab"], n_ctx=64, gate_thr=thr)
    near = np.full(s["n_layers"], -1.0, np.float32)
    idx = np.full(s["n_layers"], -1, np.int32)
    if log:
        om.m.gate_near = near.ctypes.data
        om.m.gate_near_idx = idx.ctypes.data
    if flip is not None:
        cols = [flip] if np.isscalar(flip) else list(flip)
        om.m.flip = len(cols)
        for f, col in enumerate(cols):
            om.m.flip_tok[f], om.m.flip_layer[f], om.m.flip_col[f] = 0, 0, col
    out = np.zeros(s["n_vocab"], np.float32)
    assert O.or_forward(om.ptr, np.array([tok], np.int32), 1, out) == 0
    return out, near, idx


def test_flip_of_computed_column_equals_zeroed_up_row(tmp_path):
    raw = model(tmp_path)
    col = 17
    got, _, _ = run(raw, 5, 0.0, flip=col)
    z = dict(raw)
    up = raw["blk.0.ffn_up.weight"].copy()
    up[col]["d"] = 0
    z["blk.0.ffn_up.weight"] = up
    want, _, _ = run(z, 5, 0.0)
    assert np.array_equal(got, want)
    base, _, _ = run(raw, 5, 0.0)
    assert not np.array_equal(base, got)


def test_two_flips_equal_two_zeroed_up_rows(tmp_path):
    raw = model(tmp_path)
    cols = [17, 60]
    got, _, _ = run(raw, 5, 0.0, flip=cols)
    z = dict(raw)
    up = raw["blk.0.ffn_up.weight"].copy()
    for col in cols:
        up[col]["d"] = 0
    z["blk.0.ffn_up.weight"] = up
    want, _, _ = run(z, 5, 0.0)
    assert np.array_equal(got, want)
    one, _, _ = run(raw, 5, 0.0, flip=cols[0])
    assert not np.array_equal(one, got)


def test_flip_of_skipped_column_equals_single_unskipped_row(tmp_path):
    raw = model(tmp_path)
    col = 42
    got, _, _ = run(raw, 9, 1e9, flip=col)    # every column skipped but col
    z = dict(raw)
    up = raw["blk.0.ffn_up.weight"].copy()
    keep = up[col].copy()
    up["d"] = 0
    up[col] = keep
    z["blk.0.ffn_up.weight"] = up
    want, _, _ = run(z, 9, 0.0)               # no skipping, other rows zero
    assert np.array_equal(got, want)


def test_gate_log_names_the_column_nearest_the_threshold(tmp_path):
    raw = model(tmp_path)
    s = SHAPE
    tok, thr = 11, 0.01
    _, near, idx = run(raw, tok, thr, log=True)
    # numpy float64: embedding row, RMSNorm (F32 ones), gate GEMV, silu
    x = N.q4_values(raw["token_embd.weight"])[tok]
    w = raw["blk.0.ffn_norm.weight"].astype(np.float64)
    # the FFN input is x + attention(x); recompute the attention output from
    # the oracle itself is not independent, so pin on a model without the
    # attention contribution: one token attends only to itself, out = v
    xn = x / np.sqrt(np.mean(x * x) + 1e-5) * raw["blk.0.attn_norm.weight"]
    v = N.q4_values(raw["blk.0.attn_v.weight"]) @ xn
    hd = s["n_embd"] // s["n_heads"]
    grp = s["n_heads"] // s["n_kv_heads"]
    att = np.concatenate([v[(h // grp) * hd:(h // grp + 1) * hd] for h in range(s["n_heads"])])
    x1 = x + N.q4_values(raw["blk.0.attn_output.weight"]) @ att
    xn1 = x1 / np.sqrt(np.mean(x1 * x1) + 1e-5) * w
    g = N.q4_values(raw["blk.0.ffn_gate.weight"]) @ xn1
    sg = g / (1.0 + np.exp(-g))
    dist = np.abs(np.abs(sg) - thr)
    order = np.argsort(dist)
    assert dist[order[1]] - dist[order[0]] > 1e-5     # a unique nearest column
    assert idx[0] == order[0]
    assert abs(near[0] - dist[order[0]]) < 1e-5
