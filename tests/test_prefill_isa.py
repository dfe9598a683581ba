"""ISA checks of the large-M kernels (CPU; needs hipcc, no GPU).

sm24_prefill_kernel (2:4) and marlin_dense_prefill_kernel (dense) issue their MFMAs
as inline assembly (accumulators in AGPRs), so the compiler's hazard recognizer does
not guard them.  These tests compile the kernels to gfx950 assembly and check, on
every instantiation, the two rules the kernels rely on (the wait states hipcc itself
inserts around the MFMA builtins):

* a VALU write of a register that an smfmac reads (A, B, index or accumulator)
  lies at least 2 wait states before it;
* nothing reads an smfmac's accumulator within ACC_READ_WAIT_STATES (20) wait states
  after it, except a following smfmac on the same accumulator (hardware-forwarded).

The window is the CDNA3/CDNA4 ISA's required-independent-instructions rule for an XDL
(matrix) instruction followed by a VALU, memory or export read of its result
(NumPasses + 3 wait states, one more on gfx950 for instructions of more than two
passes; LLVM's GCNHazardRecognizer encodes the table as
GFX940_XDL_N_PassWriteVgprVALUMemExpReadWaitStates), taken at its largest, 16 passes:
20 wait states cover every MFMA and smfmac whatever its pass count, so a drain cut
below that fails here.  The kernels drain 24 (three s_nop 7).

A planted violation is caught (test_checker_catches_planted_hazards), so a pass
means something.  They also check that the accumulators live in AGPRs and nothing
spills.
"""
import os
import pathlib
import re
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
SRC = ROOT / "csed499ii_amd" / "csrc" / "sm24_prefill.hip"
DENSE_SRC = ROOT / "csed499ii_amd" / "csrc" / "marlin_dense_prefill.hip"
MFMA = ("v_smfmac", "v_mfma")
ACC_READ_WAIT_STATES = 20  # XDL result -> VALU/memory read, 16-pass worst case on gfx950


def _regs(tok):
    m = re.match(r"^([va])\[(\d+):(\d+)\]$", tok)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"^([va])(\d+)$", tok)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _instructions(body):
    out = []
    for line in body.split("\n"):
        s = line.split(";")[0].strip()
        if not s or s.startswith(".") or s.endswith(":"):
            continue
        parts = s.split(None, 1)
        ops = [o.strip().split()[0] for o in parts[1].split(",") if o.strip()] if len(parts) > 1 else []
        out.append((parts[0], s, ops))
    return out


def _wait_states(op, ops):
    return int(ops[0], 0) + 1 if op == "s_nop" else 1


def hazards(body):
    """Violations of the two rules in one kernel's instruction stream (linear order,
    plus the loop tail before a loop head)."""
    ins = _instructions(body)
    labels = {}
    flat = []
    for line in body.split("\n"):
        s = line.split(";")[0].strip()
        if s.endswith(":") and not s.startswith("."):
            labels[s[:-1]] = len(flat)
        elif s and not s.startswith("."):
            parts = s.split(None, 1)
            ops = [o.strip().split()[0] for o in parts[1].split(",") if o.strip()] if len(parts) > 1 else []
            flat.append((parts[0], s, ops))
    assert len(flat) == len(ins)
    tails = {}
    for k, (op, _, ops) in enumerate(flat):
        if (op.startswith("s_cbranch") or op == "s_branch") and ops and ops[0] in labels and labels[ops[0]] <= k:
            tails[labels[ops[0]]] = k
    found = []
    for i, (op, s, ops) in enumerate(flat):
        if not op.startswith(MFMA):
            continue
        reads = set().union(*(_regs(o) for o in ops[:4]))
        window, w, j = [], 0, i - 1
        while j >= 0 and w < 2:
            window.append((flat[j], w))
            w += _wait_states(flat[j][0], flat[j][2])
            j -= 1
        if i in tails:
            w, j = 0, tails[i]
            while j > i and w < 2:
                window.append((flat[j], w))
                w += _wait_states(flat[j][0], flat[j][2])
                j -= 1
        for (pop, ps, pops), pw in window:
            if pop.startswith("v_") and not pop.startswith(MFMA) and pops and _regs(pops[0]) & reads:
                found.append(f"VALU write {pw} wait states before smfmac: {ps!r} -> {s!r}")
        dst, w, j = _regs(ops[0]), 0, i + 1
        while j < len(flat) and w < ACC_READ_WAIT_STATES:
            nop, ns, nops = flat[j]
            if nop.startswith(MFMA) and _regs(nops[0]) == dst:
                break
            if nop.startswith(("global_store", "buffer_store", "flat_store", "ds_write")):
                rd = set().union(*(_regs(o) for o in nops)) if nops else set()
            else:
                rd = set().union(*(_regs(o) for o in nops[1:])) if nops else set()
            if rd & dst:
                found.append(f"accumulator read {w} wait states after smfmac: {s!r} -> {ns!r}")
            w += _wait_states(nop, nops)
            j += 1
    return found


def _kernels(asm, name="sm24_prefill_kernel"):
    return {m.group(1): m.group(0) for m in re.finditer(r"\n(_Z\w*" + name + r"\w*):.*?s_endpgm", asm, re.S)}


def _compile(src, tmp_path_factory):
    hipcc = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not pathlib.Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / (src.stem + ".s")
    from csed499ii_amd import build
    cmd = [hipcc, *build.compile_flags(), *build.EXTRA_FLAGS.get(src.name, []), "--cuda-device-only", "-S",
           "-o", str(out), str(src)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return out.read_text()


@pytest.fixture(scope="module")
def prefill_asm(tmp_path_factory):
    return _compile(SRC, tmp_path_factory)


@pytest.fixture(scope="module")
def dense_prefill_asm(tmp_path_factory):
    return _compile(DENSE_SRC, tmp_path_factory)


def test_checker_catches_planted_hazards():
    """Planted violations are caught: a VALU write one wait state before an smfmac,
    an accumulator read right after one, and a read after an 8-wait-state drain
    (enough for a two-pass XDL op, not for the 20 the rule asks of any pass count);
    a read after the kernels' 24-wait-state drain passes."""
    planted = """
\tv_pk_mul_f16 v9, v1, v2
\ts_nop 0
\tv_smfmac_f32_32x32x32_f16 a[0:15], v[8:11], v[20:27], v30
\tv_accvgpr_read_b32 v0, a1
\tv_mov_b32_e32 v30, 0
\ts_nop 1
\tv_smfmac_f32_32x32x32_f16 a[16:31], v[8:11], v[20:27], v30
\ts_nop 7
\tglobal_store_dwordx4 v0, a[16:19], s[0:1]
"""
    found = hazards(planted)
    assert len(found) == 3, found
    assert "1 wait states before" in found[0] and "accumulator read 0" in found[1]
    assert "accumulator read 8 wait states" in found[2]
    drained = planted.replace("\ts_nop 7\n", "\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n")
    assert len(hazards(drained)) == 2


def test_prefill_smfmac_hazards(prefill_asm):
    kernels = _kernels(prefill_asm)
    # grouped and per-column scales: 512-column tiles of 128 and 64 rows (8 waves) and
    # the narrow 256-column, 128-row tile (4 waves)
    assert len(kernels) == 6
    for name, body in kernels.items():
        # four unrolled k-steps of 16 (128 rows) or 8 (64 rows) smfmacs
        assert sum(1 for l in body.split("\n") if "v_smfmac" in l) >= (32 if "ELi2E" in name else 64), name
        assert hazards(body) == [], name


def test_prefill_registers(prefill_asm):
    # no scratch; 128 (128-row tiles) or 64 (64-row tiles) accumulator registers in
    # AGPRs; architectural VGPRs (the accumulators' offset in the unified file) at most
    # 128 for the 8-wave tiles, so that two waves fit on a SIMD, and at most 256 for the
    # 4-wave narrow tile (one wave per SIMD)
    seen = 0
    for m in re.finditer(r"\.amdhsa_kernel (\S+)(.*?)\.end_amdhsa_kernel", prefill_asm, re.S):
        name, body = m.group(1), m.group(2)
        assert int(re.search(r"\.amdhsa_private_segment_fixed_size\s+(\d+)", body).group(1)) == 0, name
        waves = int(re.search(r"kernelILb[01]ELi\dELi(\d)E", name).group(1))
        arch = int(re.search(r"\.amdhsa_accum_offset\s+(\d+)", body).group(1))
        assert arch <= (128 if waves == 8 else 256), (name, arch)
        seen += 1
    assert seen == 6
    assert prefill_asm.count("; NumAgprs: 128") == 4
    assert prefill_asm.count("; NumAgprs: 64") == 2


def test_dense_prefill_mfma_hazards(dense_prefill_asm):
    kernels = _kernels(dense_prefill_asm, "marlin_dense_prefill_kernel")
    assert len(kernels) == 2  # grouped and per-column scales
    for name, body in kernels.items():
        assert sum(1 for l in body.split("\n") if "v_mfma_f32_32x32x16_f16" in l) >= 128, name
        assert hazards(body) == [], name


def test_dense_prefill_registers(dense_prefill_asm):
    for m in re.finditer(r"\.amdhsa_kernel (\S+)(.*?)\.end_amdhsa_kernel", dense_prefill_asm, re.S):
        body = m.group(2)
        assert int(re.search(r"\.amdhsa_private_segment_fixed_size\s+(\d+)", body).group(1)) == 0, m.group(1)
    assert dense_prefill_asm.count("; NumAgprs: 128") == 2
    for v in re.findall(r"; NumVgprs: (\d+)", dense_prefill_asm):
        assert int(v) <= 128
