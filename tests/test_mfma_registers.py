"""No MFMA in the shipped library writes a VGPR destination that overlaps its
own A or B source registers.

In the VGPR form (results in VGPRs instead of accumulation registers) such
an MFMA computes wrong values on gfx950, and the compiler produces one
whenever a source dies at the MFMA that starts a chain.  The kernels keep
their sources live past their MFMAs (empty asm statements); this test reads
the gfx950 code objects out of libveltrix_amd.so (clang-offload-bundler on
each bundle of the .hip_fatbin section, then llvm-objdump) and checks every
v_mfma instruction's register ranges.  CPU only: it disassembles code built
in this repository."""
import os
import re
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(ROOT, "veltrix-engine_amd", "lib", "libveltrix_amd.so")
LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _regs(tok):
    tok = tok.strip(",")
    m = re.match(r"([va])\[(\d+):(\d+)\]$", tok)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)$", tok)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _mfma_lines(tmp_path):
    sec = tmp_path / "fatbin.bin"
    subprocess.run([f"{LLVM}/llvm-objcopy", "-O", "binary", "--only-section=.hip_fatbin", LIB, str(sec)],
                   check=True)
    data = sec.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    assert starts, "no offload bundle in the library"
    lines = []
    for i, s in enumerate(starts):
        chunk = tmp_path / f"b{i}.bin"
        chunk.write_bytes(data[s:starts[i + 1] if i + 1 < len(starts) else len(data)])
        co = tmp_path / f"b{i}.co"
        r = subprocess.run([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o", f"--input={chunk}",
                            "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"],
                           capture_output=True, text=True)
        if r.returncode != 0 or not co.exists() or co.stat().st_size == 0:
            continue
        out = subprocess.run([f"{LLVM}/llvm-objdump", "-d", str(co)], check=True, capture_output=True,
                             text=True).stdout
        lines += [ln.split("//")[0].strip() for ln in out.splitlines() if "v_mfma" in ln]
    return lines


@pytest.mark.skipif(not os.path.exists(LIB) or not os.path.exists(f"{LLVM}/clang-offload-bundler"),
                    reason="library not built or ROCm LLVM tools missing")
def test_no_mfma_destination_overlaps_its_sources(tmp_path):
    lines = _mfma_lines(tmp_path)
    assert len(lines) > 100, f"only {len(lines)} MFMA instructions found"
    bad = []
    for ln in lines:
        toks = ln.replace(",", " ").split()
        op = next(i for i, t in enumerate(toks) if t.startswith("v_mfma"))
        dst, a, b = _regs(toks[op + 1]), _regs(toks[op + 2]), _regs(toks[op + 3])
        if dst & (a | b):
            bad.append(ln)
    print(f"{len(lines)} MFMA instructions checked")
    assert not bad, f"{len(bad)} MFMAs write over their own sources, e.g. {bad[:3]}"
