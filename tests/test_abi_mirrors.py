"""The ctypes mirrors of the C-ABI structs (tests and bench.py) against the
headers: size and member offsets as the C compiler lays them out.  A mirror
shorter than its struct is memory corruption, not a test failure, once the
library writes the whole struct (vxh_qmat_alloc clears it), so every mirror
is checked here, on the CPU, before any GPU test uses it."""
import ctypes as C
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, ROOT)

import _native as N  # noqa: E402

# C type -> members whose offsets are checked (all of them)
STRUCTS = {
    "vxh_qmat": ["type", "n_rows", "n_cols", "n_pairs", "qs", "d", "cached", "tq", "td"],
    "vxh_panel": ["data", "corr", "rscale", "xs", "M", "K", "avx2", "rs_ld"],
    "vxh_workspace": ["acc", "acc_elems", "part", "part_floats"],
    "vxh_pro": ["kind", "x", "ldx", "src", "ld_src", "w", "x_out", "ld_xout", "ss", "ss_in", "ss_K", "thr",
                "clear", "n_clear", "part", "n_chunks", "n_heads", "n_kv_heads", "head_dim"],
    "vx_model_options": ["q4_kernel", "attn_cap", "ffn_gate_threshold", "fused", "pro_max_rows", "kv_half",
                         "prefill_min_rows"],
    "vx_synth_spec": ["seed", "std", "matrix_type", "embd_type", "output_type"],
    "vx_gemm_profile": ["launches", "ms", "bytes", "flops"],
    "vx_speculative_stats": ["rounds", "drafted", "accepted", "emitted", "verify_ms", "draft_ms", "prefill_ms"],
    "vxh_vocab_ws": ["part", "cnt", "stats", "max_rows"],
}


@pytest.fixture(scope="module")
def layout(tmp_path_factory):
    d = tmp_path_factory.mktemp("abi")
    src = ['#include <stdio.h>', '#include <stddef.h>', '#include "vxh.h"', '#include "veltrix_gpu.h"',
           "int main(void) {"]
    for t, members in STRUCTS.items():
        src.append(f'printf("{t} size %zu\\n", sizeof({t}));')
        for m in members:
            src.append(f'printf("{t} {m} %zu\\n", offsetof({t}, {m}));')
    src.append("return 0; }")
    c = d / "abi.c"
    c.write_text("\n".join(src) + "\n")
    exe = d / "abi"
    subprocess.run(["gcc", "-std=gnu11", "-I", os.path.join(ROOT, "include"), str(c), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    lay = {}
    for line in out.splitlines():
        t, m, v = line.split()
        lay[(t, m)] = int(v)
    return lay


def mirrors():
    import bench
    import test_gpu_gemm
    import test_gpu_pro
    import test_zz_no_alloc
    return [
        ("vxh_qmat", test_gpu_gemm._QMat), ("vxh_qmat", test_gpu_pro.Qmat), ("vxh_qmat", test_zz_no_alloc.QMat),
        ("vxh_qmat", bench._QMat),
        ("vxh_panel", test_gpu_gemm._Panel), ("vxh_panel", test_zz_no_alloc.Panel), ("vxh_panel", bench._Panel),
        ("vxh_workspace", test_gpu_pro.Workspace), ("vxh_workspace", test_zz_no_alloc.Workspace),
        ("vxh_pro", test_gpu_pro.Pro), ("vxh_pro", bench._Pro),
        ("vx_model_options", N.VxModelOptions), ("vx_synth_spec", N.VxSynthSpec),
        ("vx_gemm_profile", N.VxGemmProfile), ("vx_speculative_stats", N.VxSpecStats),
        ("vxh_vocab_ws", N.VxhVocabWs),
    ]


def test_ctypes_mirrors_match_the_headers(layout):
    bad = []
    for ctype, cls in mirrors():
        name = f"{cls.__module__}.{cls.__name__}"
        if C.sizeof(cls) != layout[(ctype, "size")]:
            bad.append(f"{name}: size {C.sizeof(cls)} != sizeof({ctype}) {layout[(ctype, 'size')]}")
        for m in STRUCTS[ctype]:
            if not hasattr(cls, m):
                bad.append(f"{name}: no member {m}")
            elif getattr(cls, m).offset != layout[(ctype, m)]:
                bad.append(f"{name}.{m}: offset {getattr(cls, m).offset} != {layout[(ctype, m)]}")
    assert not bad, "\n".join(bad)
