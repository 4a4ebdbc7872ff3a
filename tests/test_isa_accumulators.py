"""Guard on the inline-asm MFMA accumulators of the dq and dk/dv kernels (CPU).

The dq and dk/dv kernels accumulate dQ / dK / dV in AGPRs through an inline-
asm MFMA (``mfma32_agpr`` in logo_amd/csrc/common.hpp) that the compiler
cannot see into: it supplies no wait states for it and does not know the
instruction writes its accumulator.  Correctness therefore needs (1) no copy
of those accumulator registers (``v_accvgpr_read`` / ``_mov`` / ``_write``)
anywhere between the first and the last such MFMA of a kernel, i.e. inside
its MFMA loops, where a copy would read the register before the MFMA wrote
it; and (2) every read of them after the loops preceded by the drain
(``agpr_acc_drain``: two ``s_nop 15``) rather than directly by an MFMA.

This test extracts the gfx950 code object from the in-tree
``logo_amd/liblogo_hip.so`` (built here from source), disassembles it with
ROCm's llvm-objdump and checks both rules for every sq_dq64 / sq_dkv
instantiation.  Planted mistakes on synthetic listings show the checker
catches both kinds of violation.
"""

import os
import re
import shutil
import struct
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "logo_amd", "liblogo_hip.so")
LLVM = "/opt/rocm/llvm/bin"
BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"

_ACC_DST = re.compile(r"v_mfma_\S+\s+a\[(\d+):(\d+)\]")
_KERNEL = re.compile(r"^[0-9a-f]+ <(_ZN4logo\S+)>:$")


def _regs(tok):
    tok = tok.rstrip(",")
    m = re.fullmatch(r"a\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"a(\d+)", tok)
    return {int(m.group(1))} if m else set()


def check_accumulators(lines):
    """Violations (line index, text) of the two rules in one kernel's listing."""
    acc, mfma_at = set(), []
    for n, line in enumerate(lines):
        m = _ACC_DST.search(line)
        if m:
            acc.update(range(int(m.group(1)), int(m.group(2)) + 1))
            mfma_at.append(n)
    if not mfma_at:
        return []
    first, last = mfma_at[0], mfma_at[-1]
    bad = []
    for n, line in enumerate(lines):
        code = line.split("//")[0].split()
        if not code or code[0].startswith("v_mfma"):
            continue
        touched = set().union(*(_regs(t) for t in code[1:]))
        if not (touched & acc):
            continue
        if first < n < last:
            bad.append((n, "inside the MFMA range: " + line.strip()))
            continue
        reads = code[0] in ("v_accvgpr_read_b32", "v_accvgpr_mov_b32") and (_regs(code[-1]) & acc)
        if not reads:
            continue
        # walk back to the nearest accumulator MFMA or drain
        k, nops = n - 1, 0
        while k >= 0:
            prev = lines[k].split("//")[0].strip()
            if _ACC_DST.search(prev):
                bad.append((n, "read with no drain after an MFMA: " + line.strip()))
                break
            nops = nops + 1 if prev == "s_nop 15" else 0
            if nops == 2:
                break
            k -= 1
    return bad


def _gfx950_objects(lib_path, tmp_path):
    section = tmp_path / "hip_fatbin.bin"
    subprocess.run([f"{LLVM}/llvm-objcopy", "-O", "binary", "--only-section=.hip_fatbin", lib_path, str(section)],
                   capture_output=True, check=True)
    out = section.read_bytes()
    objs, pos = [], 0
    while True:
        i = out.find(BUNDLE_MAGIC, pos)
        if i < 0:
            return objs
        (count,) = struct.unpack_from("<Q", out, i + 24)
        off = i + 32
        for _ in range(count):
            eo, es, ts = struct.unpack_from("<QQQ", out, off)
            off += 24
            triple = out[off:off + ts].decode()
            off += ts
            if "gfx950" in triple:
                objs.append(out[i + eo:i + eo + es])
        pos = i + len(BUNDLE_MAGIC)


def _kernel_listings(tmp_path):
    listings = {}
    for j, obj in enumerate(_gfx950_objects(LIB, tmp_path)):
        if b"sq_dkv_kernel" not in obj and b"sq_dq64_kernel" not in obj:
            continue
        path = tmp_path / f"co{j}.o"
        path.write_bytes(obj)
        text = subprocess.run([f"{LLVM}/llvm-objdump", "-d", "--mcpu=gfx950", str(path)], capture_output=True,
                              text=True, check=True).stdout
        name = None
        for line in text.splitlines():
            m = _KERNEL.match(line)
            if m:
                name = m.group(1)
                listings[name] = []
            elif name is not None:
                listings[name].append(line)
    return listings


@pytest.mark.skipif(not (os.path.exists(LIB) and shutil.which(f"{LLVM}/llvm-objdump")),
                    reason="needs the built library and ROCm's llvm-objdump")
def test_asm_accumulators_are_not_copied_inside_mfma_loops(tmp_path):
    listings = _kernel_listings(tmp_path)
    kernels = [k for k in listings if "sq_dq64_kernel" in k or "sq_dkv_kernel" in k]
    # bf16: {dq, dkv} x D {64, 128} x sparse x window; fp16: {dq, dkv} x D, sparse without window
    assert len(kernels) == 20, sorted(listings)
    for name in kernels:
        lines = listings[name]
        assert any(_ACC_DST.search(line) for line in lines), f"{name}: no AGPR-accumulator MFMA found"
        # the element type's MFMA, and no other (an fp16 kernel on the bf16 unit, or the reverse)
        want = "f16" if "IDF16_" in name else "bf16"
        ops = {m.group(1) for m in re.finditer(r"v_mfma_f32_32x32x16_(b?f16)", "\n".join(lines))}
        assert ops == {want}, f"{name}: MFMA types {sorted(ops)}, expected {want}"
        bad = check_accumulators(lines)
        assert not bad, f"{name}: " + "; ".join(f"line {n}: {t[:100]}" for n, t in bad[:5])


_GOOD = """\
	v_accvgpr_write_b32 a0, 0
	s_nop 2
	v_mfma_f32_32x32x16_bf16 a[0:15], v[2:5], v[6:9], a[0:15]
	v_mfma_f32_32x32x16_bf16 v[20:35], v[2:5], v[6:9], 0
	s_nop 2
	v_mfma_f32_32x32x16_bf16 a[0:15], v[2:5], v[6:9], a[0:15]
	s_nop 15
	s_nop 15
	v_accvgpr_read_b32 v40, a3
""".splitlines()


def test_checker_accepts_a_clean_listing():
    assert check_accumulators(_GOOD) == []


def test_checker_flags_a_copy_inside_the_loop():
    bad = list(_GOOD)
    bad.insert(4, "\tv_accvgpr_mov_b32 a200, a5")
    found = check_accumulators(bad)
    assert found and "inside the MFMA range" in found[0][1]


def test_checker_flags_a_read_without_drain():
    bad = [line for line in _GOOD if "s_nop 15" not in line]
    found = check_accumulators(bad)
    assert found and "no drain" in found[0][1]
