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


def _vregs(tok):
    tok = tok.rstrip(",")
    m = re.fullmatch(r"-?v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"-?v(\d+)", tok)
    return {int(m.group(1))} if m else set()


# A VALU write of an MFMA's A or B operand needs wait states before the MFMA
# (two on the gfx9 MFMA parts; three are required here).  The compiler adds
# them for its own MFMAs but not for the inline-asm accumulator MFMAs without
# a leading s_nop (mfma32_agpr_ready), so for those the distance is checked.
OPERAND_WAIT_STATES = 3


def check_operand_distance(lines):
    """Violations (line index, text): an accumulator MFMA whose A or B
    VGPRs a VALU instruction wrote within OPERAND_WAIT_STATES wait states
    before it, on any control-flow path into it (each instruction is one
    wait state, s_nop N is N + 1).  The walk follows _flow's predecessors,
    so a write at the end of a loop body that reaches an MFMA at the loop
    head through the back edge is seen too."""
    code, preds = _flow(lines)
    bad = []
    for n, c in enumerate(code):
        if not (c and c[0].startswith("v_mfma") and len(c) >= 4 and _ACC_DST.search(lines[n])):
            continue
        srcs = _vregs(c[2]) | _vregs(c[3])
        # backward search over (line, wait states between it and the MFMA)
        stack, seen = [(k, 0) for k in preds[n]], set()
        while stack:
            k, waits = stack.pop()
            if (k, waits) in seen:
                continue
            seen.add((k, waits))
            p = code[k]
            if not p or p[0].startswith((".", ";")) or p[0].endswith(":"):
                stack.extend((q, waits) for q in preds[k])
                continue
            if p[0].startswith("v_") and not p[0].startswith(("v_mfma", "v_accvgpr_write")) and len(p) > 1:
                if _vregs(p[1]) & srcs:
                    bad.append((n, "operand written %d wait state(s) before: %s" % (waits, lines[k].strip())))
                    break
            waits += int(p[1]) + 1 if p[0] == "s_nop" and len(p) > 1 else 1
            if waits < OPERAND_WAIT_STATES:
                stack.extend((q, waits) for q in preds[k])
    return bad


_ADDR = re.compile(r"//\s*([0-9A-Fa-f]+):")
_UNCOND = ("s_branch", "s_setpc_b64", "s_endpgm")


def _flow(lines):
    """(code, predecessors) per line of a kernel listing: the instruction
    text, and the indices of the lines control can come from (the line
    before unless it ends in an unconditional jump, and every branch whose
    target, PC + 4 + 4 * simm16, is this line's address).  Listings without
    addresses (the synthetic ones below) fall through line by line."""
    code = [line.split("//")[0].split() for line in lines]
    addr = {}
    for n, line in enumerate(lines):
        m = _ADDR.search(line)
        if m:
            addr[int(m.group(1), 16)] = n
    preds = [[] for _ in lines]
    for n, c in enumerate(code):
        if n + 1 < len(lines) and not (c and c[0] in _UNCOND):
            preds[n + 1].append(n)
        if c and c[0].startswith(("s_branch", "s_cbranch")) and len(c) > 1:
            m = _ADDR.search(lines[n])
            try:
                imm = int(c[1]) if not c[1].startswith("0x") else int(c[1], 16)
            except ValueError:
                continue
            if imm >= 1 << 15:
                imm -= 1 << 16
            tgt = addr.get(int(m.group(1), 16) + 4 + 4 * imm) if m else None
            if tgt is not None:
                preds[tgt].append(n)
    return code, preds


def check_accumulators_drained(lines):
    """Violations of the rule for kernels that also read or clear their
    accumulators between MFMA phases (the fused window backward stores dQ
    rows inside its walk): on every control-flow path into an instruction
    that touches registers an accumulator MFMA writes, a drain (two s_nop 15)
    lies between it and the nearest MFMA whose accumulator overlaps them
    (the asm MFMA's result is not written yet when it issues; MFMAs into
    other accumulators do not matter)."""
    acc = set()
    dst = []
    for line in lines:
        m = _ACC_DST.search(line)
        r = set(range(int(m.group(1)), int(m.group(2)) + 1)) if m else set()
        acc |= r
        dst.append(r)
    code, preds = _flow(lines)
    bad = []
    for n, c in enumerate(code):
        if not c or c[0].startswith("v_mfma"):
            continue
        touched = set().union(*(_regs(t) for t in c[1:])) & acc
        if not touched:
            continue
        # backward search over (line, consecutive s_nop 15 seen after it)
        stack, seen, hit = [(p, 0) for p in preds[n]], set(), False
        while stack and not hit:
            k, nops = stack.pop()
            if (k, nops) in seen:
                continue
            seen.add((k, nops))
            if dst[k] & touched:
                hit = True
                break
            nops = nops + 1 if code[k] == ["s_nop", "15"] else 0
            if nops == 2:
                continue
            stack.extend((p, nops) for p in preds[k])
        if hit:
            bad.append((n, "accumulator touched with no drain after an MFMA: " + lines[n].strip()))
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
        if b"sq_dkv_kernel" not in obj and b"sq_dq64_kernel" not in obj and b"swa_bwd_kernel" not in obj:
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
        bad = check_operand_distance(lines)
        assert not bad, f"{name}: " + "; ".join(f"line {n}: {t[:100]}" for n, t in bad[:5])


@pytest.mark.skipif(not (os.path.exists(LIB) and shutil.which(f"{LLVM}/llvm-objdump")),
                    reason="needs the built library and ROCm's llvm-objdump")
def test_window_backward_accumulators_are_drained_before_use(tmp_path):
    listings = _kernel_listings(tmp_path)
    kernels = [k for k in listings if "swa_bwd_kernel" in k]
    assert len(kernels) == 2, sorted(listings)  # D = 64, 128
    for name in kernels:
        lines = listings[name]
        assert any(_ACC_DST.search(line) for line in lines), f"{name}: no AGPR-accumulator MFMA found"
        bad = check_accumulators_drained(lines)
        assert not bad, f"{name}: " + "; ".join(f"line {n}: {t[:100]}" for n, t in bad[:5])
        bad = check_operand_distance(lines)
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


def test_drain_checker_accepts_reads_and_clears_after_a_drain():
    assert check_accumulators_drained(_GOOD) == []
    mid = _GOOD[:6] + ["\ts_nop 15", "\ts_nop 15", "\tv_accvgpr_read_b32 v41, a2", "\tv_accvgpr_write_b32 a2, 0"]
    assert check_accumulators_drained(mid + _GOOD[6:]) == []


def test_drain_checker_flags_a_clear_right_after_an_mfma():
    bad = _GOOD[:6] + ["\tv_accvgpr_write_b32 a2, 0"] + _GOOD[6:]
    found = check_accumulators_drained(bad)
    assert found and "no drain" in found[0][1]


def test_drain_checker_ignores_other_accumulators():
    ok = _GOOD[:6] + ["\tv_accvgpr_write_b32 a16, v3", "\ts_nop 2",
                      "\tv_mfma_f32_32x32x16_bf16 a[16:31], v[2:5], v[6:9], a[16:31]"] + _GOOD[6:]
    assert check_accumulators_drained(ok) == []


def test_operand_checker_accepts_distant_writes():
    ok = ["\tv_cvt_pk_bf16_f32 v6, v40, v41", "\tds_read_b128 v[2:5], v90", "\ts_waitcnt lgkmcnt(0)",
          "\tv_exp_f32_e64 v50, -v51", "\tv_mfma_f32_32x32x16_bf16 a[0:15], v[2:5], v[6:9], a[0:15]"]
    assert check_operand_distance(ok) == []
    assert check_operand_distance(["\tv_cvt_pk_bf16_f32 v6, v40, v41", "\ts_nop 2",
                                   "\tv_mfma_f32_32x32x16_bf16 a[0:15], v[2:5], v[6:9], a[0:15]"]) == []


def test_operand_checker_flags_a_recent_valu_write():
    bad = ["\tv_cvt_pk_bf16_f32 v7, v40, v41", "\ts_waitcnt lgkmcnt(0)",
           "\tv_mfma_f32_32x32x16_bf16 a[0:15], v[2:5], v[6:9], a[0:15]"]
    found = check_operand_distance(bad)
    assert found and "operand written" in found[0][1]
    # a VGPR-result MFMA is the compiler's to protect, and is not checked
    assert check_operand_distance(["\tv_cvt_pk_bf16_f32 v7, v40, v41",
                                   "\tv_mfma_f32_32x32x16_bf16 v[20:35], v[2:5], v[6:9], 0"]) == []


# A loop with addresses: the MFMA at the loop head (0x10) is reached from the
# line before it and, through the back edge (s_cbranch_scc1 at 0x1c, simm16
# -4: 0x1c + 4 - 16 = 0x10), from the end of the loop body.
_LOOP = """\
	v_mov_b32 v8, 0 // 000000000008: 0
	s_nop 4 // 00000000000C: 0
	v_mfma_f32_32x32x16_bf16 a[0:15], v[2:5], v[6:9], a[0:15] // 000000000010: 0
	s_add_i32 s4, s4, 1 // 000000000014: 0
	{last} // 000000000018: 0
	s_cbranch_scc1 65532 // 00000000001C: 0
	s_endpgm // 000000000020: 0
"""


def test_operand_checker_follows_the_loop_back_edge():
    # the write at the loop end is one wait state before the loop head's MFMA
    found = check_operand_distance(_LOOP.format(last="v_cvt_pk_bf16_f32 v7, v40, v41").splitlines())
    assert found and "operand written 1 wait state" in found[0][1]
    # a write to another register there is fine, and so is the straight-line
    # entry (s_nop 4 between the v8 write and the MFMA)
    assert check_operand_distance(_LOOP.format(last="v_cvt_pk_bf16_f32 v70, v40, v41").splitlines()) == []
