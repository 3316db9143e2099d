"""CPU checks on the gfx950 assembly of the HIP kernels.

Instructions issued through inline asm (LDS operand reads with explicit waits,
the bf16 dot2 instruction) are scheduled by the compiler without knowing their
latencies, so two mistakes compile silently and only show up as wrong numbers
on the GPU:

* a register written by an inline ``ds_read`` is read, copied or overwritten
  before the ``s_waitcnt lgkmcnt`` that covers the read (the copy sees stale
  data);
* the result of ``v_dot2_f32_bf16`` (written through the dot pipeline) is read
  by a different VALU instruction fewer than 3 wait states later.

These tests compile each kernel source to device assembly with the library's own
flags and scan it for both.  A third check guards a performance property: the
prefill kernel's MFMA operand ring relies on the compiler counting LDS reads in
issue order (``s_waitcnt lgkmcnt(N)`` with N > 0 before each MFMA).  A
global->LDS copy that the compiler can see anywhere in the loop makes it wait
for every outstanding LDS read (``lgkmcnt(0)``) instead, which still computes
the right result but exposes the full LDS latency before each MFMA.  The scanners are first run on small snippets in
which the mistake is planted, so a scanner that finds nothing is known to be
able to find something.
"""
import os
import re
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "atflash-kernel_amd")

_REG = re.compile(r"\b([va])(\d+)\b|\b([va])\[(\d+):(\d+)\]")


def _regs(text):
    out = set()
    for m in _REG.finditer(text):
        if m.group(1):
            out.add((m.group(1), int(m.group(2))))
        else:
            out.update((m.group(3), r) for r in range(int(m.group(4)), int(m.group(5)) + 1))
    return out


def _instructions(asm):
    """(line number, instruction text) for every instruction, comments dropped."""
    out = []
    for i, raw in enumerate(asm.split("\n"), 1):
        s = raw.split(";")[0].strip()
        if s and not s.startswith(".") and not s.endswith(":"):
            out.append((i, s))
    return out


def lds_read_hazards(asm):
    """Instructions touching the destination of an LDS read that no
    s_waitcnt lgkmcnt has retired yet (linear scan; LDS and scalar-memory
    operations retire in issue order for this purpose)."""
    pending, found = [], []
    for i, s in _instructions(asm):
        op = s.split()[0]
        args = s[len(op):]
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", args)
            if m:
                n = int(m.group(1))
                pending = pending[len(pending) - n:] if 0 < n < len(pending) else ([] if n == 0 else pending)
            continue
        touched = _regs(args)
        for ln, dst in pending:
            if dst and touched & dst:
                found.append((i, s, ln))
        if op.startswith(("ds_read", "ds_load")):
            pending.append((i, _regs(args.split(",")[0])))
        elif op.startswith(("ds_", "s_load", "s_buffer_load")):
            pending.append((i, None))
    return found


def dot_hazards(asm, need=3):
    """Reads of a v_dot2 result, other than as the accumulator of the next dot
    of the same opcode, within `need` wait states of the write."""
    ins = _instructions(asm)
    found = []
    for j, (i, s) in enumerate(ins):
        if not s.startswith("v_dot2"):
            continue
        dst = s.split()[1].rstrip(",")
        ws = 0
        for i2, s2 in ins[j + 1:]:
            op2 = s2.split()[0]
            if op2 == "s_nop":
                ws += int(s2.split()[1], 0) + 1
            else:
                ops = [o.strip() for o in s2[len(op2):].split(",")]
                srcs = ops[1:] if op2.startswith("v_") else ops
                if dst in srcs:
                    if not (op2 == s.split()[0] and srcs.index(dst) == len(srcs) - 1):
                        found.append((i2, s2, i))
                    break
                if ops and ops[0] == dst:
                    break
                ws += 1
            if ws >= need:
                break
    return found


# ------------------------------------------------------------ scanner self-tests

def test_lds_scanner_finds_a_copy_before_the_wait():
    bad = """
        ds_read_b128 v[4:7], v1 offset:0
        v_mov_b64_e32 v[20:21], v[4:5]
        s_waitcnt lgkmcnt(0)
    """
    good = """
        ds_read_b128 v[4:7], v1 offset:0
        ds_read_b128 v[8:11], v1 offset:512
        s_waitcnt lgkmcnt(1)
        v_mov_b64_e32 v[20:21], v[4:5]
        s_waitcnt lgkmcnt(0)
        v_mov_b64_e32 v[22:23], v[8:9]
    """
    early = """
        ds_read_b128 v[4:7], v1 offset:0
        ds_read_b128 v[8:11], v1 offset:512
        s_waitcnt lgkmcnt(1)
        v_mov_b64_e32 v[22:23], v[8:9]
    """
    assert len(lds_read_hazards(bad)) == 1
    assert lds_read_hazards(good) == []
    assert len(lds_read_hazards(early)) == 1


def test_dot_scanner_finds_an_early_read():
    bad = """
        v_dot2_f32_bf16 v10, v2, v3, v10
        v_add_f32_e32 v11, v10, v11
    """
    chained = """
        v_dot2_f32_bf16 v10, v2, v3, v10
        v_dot2_f32_bf16 v10, v4, v3, v10
        s_nop 4
        v_add_f32_e32 v11, v10, v11
    """
    as_source_ab = """
        v_dot2_f32_bf16 v10, v2, v3, v10
        v_dot2_f32_bf16 v12, v10, v3, v12
    """
    assert len(dot_hazards(bad)) == 1
    assert dot_hazards(chained) == []
    assert len(dot_hazards(as_source_ab)) == 1


# ------------------------------------------------------------ the kernels

def lds_waits_before_mfma(asm, kernel):
    """For each MFMA of `kernel`, the smallest lgkmcnt waited for since the
    previous MFMA (None: no LDS wait)."""
    start = asm.index(kernel + ":")
    body = asm[start:asm.index("s_endpgm", start)]
    out, cur = [], None
    for _, s in _instructions(body):
        m = re.match(r"s_waitcnt.*lgkmcnt\((\d+)\)", s)
        if m:
            cur = int(m.group(1)) if cur is None else min(cur, int(m.group(1)))
        if s.startswith("v_mfma"):
            out.append(cur)
            cur = None
    return out


def longest_pipelined_run(waits, depth=3):
    """Longest run of consecutive MFMAs waiting for at most all but `depth`
    outstanding LDS reads (or none)."""
    best = run = 0
    for w in waits:
        run = run + 1 if (w is None or w >= depth) else 0
        best = max(best, run)
    return best


def test_wait_scanner_tells_pipelined_from_drained_reads():
    mf = "v_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]"
    ring = "k:\n" + "".join(f"  ds_read_b128 v[{24 + 4 * (i % 6)}:{27 + 4 * (i % 6)}], v40\n"
                             "  s_waitcnt lgkmcnt(5)\n  " + mf + "\n" for i in range(16)) + "  s_endpgm\n"
    drained = ring.replace("lgkmcnt(5)", "lgkmcnt(0)")
    assert longest_pipelined_run(lds_waits_before_mfma(ring, "k")) == 16
    assert longest_pipelined_run(lds_waits_before_mfma(drained, "k")) == 0


def _hipcc_or_skip():
    sys.path.insert(0, PKG)
    import build as B  # atflash-kernel_amd/build.py
    if not os.path.exists(B.HIPCC) and shutil.which(B.HIPCC) is None:
        pytest.skip("hipcc not available")
    return B


@pytest.fixture(scope="module")
def kernel_asm(tmp_path_factory):
    B = _hipcc_or_skip()
    out = {}
    tmp = tmp_path_factory.mktemp("asm")
    for src in B.sources():
        if not src.endswith(".hip"):
            continue
        dst = os.path.join(tmp, os.path.basename(src) + ".s")
        flags = [f for f in B.COMMON if not f.startswith("-Rpass")]
        cmd = [B.HIPCC, *flags, "-I", B.CSRC, "--cuda-device-only", "-S", src, "-o", dst]
        p = subprocess.run(cmd, capture_output=True, text=True)
        assert p.returncode == 0, p.stderr
        with open(dst) as f:
            out[os.path.basename(src)] = f.read()
    assert "atf_prefill.hip" in out and "atf_decode.hip" in out
    return out


def test_kernel_sources_assemble(tmp_path):
    """The `-S` listing above is never run through the assembler, so an inline
    assembly operand the assembler rejects (a vector register where the
    instruction needs a scalar one) only shows when an object is built: every
    kernel source is assembled to a device object here."""
    B = _hipcc_or_skip()
    flags = [f for f in B.COMMON if not f.startswith("-Rpass")]
    for src in B.sources():
        if not src.endswith(".hip"):
            continue
        dst = os.path.join(tmp_path, os.path.basename(src) + ".o")
        p = subprocess.run([B.HIPCC, *flags, "-I", B.CSRC, "--cuda-device-only", "-c", src, "-o", dst],
                           capture_output=True, text=True)
        assert p.returncode == 0, p.stderr[-3000:]


def test_assembling_catches_a_planted_vector_operand(tmp_path):
    """Planted: a divergent value under an "s" constraint.  The `-S` listing
    accepts it; assembling rejects it."""
    B = _hipcc_or_skip()
    src = tmp_path / "planted.hip"
    src.write_text('#include <hip/hip_runtime.h>\n'
                   '__global__ void k(int* o) {\n'
                   '  int x = threadIdx.x * 3;\n'
                   '  asm volatile("s_cmp_le_i32 %0, 1" :: "s"(x) : "scc");\n'
                   '  o[threadIdx.x] = x;\n'
                   '}\n')
    flags = [f for f in B.COMMON if not f.startswith("-Rpass")]
    listing = subprocess.run([B.HIPCC, *flags, "--cuda-device-only", "-S", str(src), "-o", str(tmp_path / "p.s")],
                             capture_output=True, text=True)
    obj = subprocess.run([B.HIPCC, *flags, "--cuda-device-only", "-c", str(src), "-o", str(tmp_path / "p.o")],
                         capture_output=True, text=True)
    assert listing.returncode == 0, listing.stderr[-2000:]
    assert obj.returncode != 0 and "invalid operand" in obj.stderr


def test_no_lds_read_hazards(kernel_asm):
    for name, asm in kernel_asm.items():
        assert lds_read_hazards(asm) == [], name


def test_no_dot_result_hazards(kernel_asm):
    for name, asm in kernel_asm.items():
        assert dot_hazards(asm) == [], name


# the two instantiations of the prefill kernel: scores scaled through Q (RoPE at
# load) and raw scores scaled in the softmax (pre-rotated Q)
PREFILL_KERNELS = ("_ZN3atf14prefill_kernelILb0EEEvNS_11PrefillArgsE", "_ZN3atf14prefill_kernelILb1EEEvNS_11PrefillArgsE")


def test_prefill_kernel_does_not_spill(kernel_asm):
    asm = kernel_asm["atf_prefill.hip"]
    # kernel metadata: one "- .agpr_count" block per kernel, holding .name and .vgpr_spill_count
    for name in PREFILL_KERNELS:
        blocks = [b for b in asm.split("  - .agpr_count:") if re.search(r"\.name:\s+" + name + r"\s", b)]
        assert len(blocks) == 1, f"{name} metadata not found"
        spill = re.search(r"\.vgpr_spill_count:\s+(\d+)", blocks[0])
        assert spill and int(spill.group(1)) == 0, name


def pipelined_runs(waits, depth=3):
    """Lengths of the maximal runs counted by longest_pipelined_run."""
    runs, run = [], 0
    for w in waits:
        if w is None or w >= depth:
            run += 1
        else:
            if run:
                runs.append(run)
            run = 0
    if run:
        runs.append(run)
    return runs


def test_prefill_operand_ring_keeps_lds_reads_in_flight(kernel_asm):
    # the PV stream of a tile pair (32 MFMAs) and the 8-level QK stream of its
    # four 32-key blocks (32 MFMAs, the ring draining over the last three) run
    # with the operand reads of several later MFMAs still outstanding
    for name in PREFILL_KERNELS:
        waits = lds_waits_before_mfma(kernel_asm["atf_prefill.hip"], name)
        assert len(waits) >= 64, name
        runs = sorted(pipelined_runs(waits), reverse=True)
        assert runs[0] >= 31, (name, runs)
        assert len(runs) >= 2 and runs[1] >= 25, (name, runs)
