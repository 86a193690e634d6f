"""The 16x16x32 GEMM cores issue their MFMAs as inline asm (so the 4-register
accumulators stay in place), which hides them from the compiler's hazard
recognizer.  The cores keep the hazards by construction (operands only from LDS
reads behind explicit waits, accumulators touched only by the MFMAs until a drain
of 32 wait states); this checks the compiled code for it: in every kernel that
instantiates the cores, no instruction other than an MFMA accumulating into the
same registers reads or writes an MFMA's destination within the next 12
instructions on any path (branches followed), for the precompiled kernels (VGPR or
AGPR accumulators) and for a generated epilogue (FusedDense + tanh-GELU).  CPU only: hipcc cross-compiles for gfx950 here."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "go-darwinml_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "--cuda-device-only", "-S"]

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")


def _regs(tok):
    """Registers named by an operand: ("v", n) for VGPRs, ("a", n) for AGPRs (the
    4-wave cores accumulate in AGPRs)."""
    tok = tok.strip()
    m = re.match(r"([va])\[(\d+):(\d+)\]$", tok)
    if m:
        return {(m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)$", tok)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _violations(asm_lines, kernel_names, window=12):
    """(MFMAs checked, offending pairs) over every control-flow path of `window`
    instructions after each 16x16x32 MFMA (branches followed to their labels)."""
    labels = {}
    for i, line in enumerate(asm_lines):
        m = re.match(r"^([.\w$]+):", line)
        if m:
            labels[m.group(1)] = i
    cur, count, bad = None, 0, []
    for i, line in enumerate(asm_lines):
        if re.match(r"^[_A-Za-z][\w.$]*:", line):
            cur = line.split(":")[0]
        if cur is None or not any(k in cur for k in kernel_names):
            continue
        s = line.strip()
        if not s.startswith("v_mfma_f32_16x16x32"):
            continue
        count += 1
        dst = _regs(s.split(None, 1)[1].split(",")[0])
        work, visited = [(i + 1, window)], set()
        while work:
            k, left = work.pop()
            while k < len(asm_lines) and left > 0:
                if (k, left) in visited:
                    break
                visited.add((k, left))
                t = asm_lines[k].strip()
                k += 1
                if not t or t.startswith((";", ".")) or re.match(r"^[.\w$]+:", t):
                    continue
                left -= 1
                parts = t.split(None, 1)
                ops = parts[1].split(",") if len(parts) > 1 else []
                if t.startswith("s_endpgm"):
                    break
                if t.startswith("s_branch"):
                    k = labels.get(ops[0].strip(), len(asm_lines))
                    continue
                if t.startswith("s_cbranch"):
                    work.append((labels.get(ops[0].strip(), len(asm_lines)), left))
                    continue
                if t.startswith("v_mfma"):
                    if _regs(ops[0]) & dst and _regs(ops[3]) != _regs(ops[0]):
                        bad.append((cur, s, t))
                    continue
                if any(_regs(o) & dst for o in ops):
                    bad.append((cur, s, t))
    return count, bad


def _compile(src, out, extra=()):
    subprocess.run([HIPCC, *FLAGS, "-I", os.path.join(ROOT, "include"), "-I", CSRC, *extra, "-o", out, src],
                   check=True, capture_output=True, timeout=600)
    with open(out) as f:
        return f.read().split("\n")


def test_precompiled_cores_keep_mfma_hazards(tmp_path):
    lines = _compile(os.path.join(CSRC, "k_gemm.hip"), str(tmp_path / "k_gemm.s"))
    count, bad = _violations(lines, ["kernel4km", "kernel8x"])
    assert count >= 2048, count  # every instantiation, unrolled
    assert not bad, bad[:5]


@pytest.mark.parametrize("case", ["gelu", "residual"])
def test_generated_epilogue_keeps_mfma_hazards(tmp_path, monkeypatch, case):
    """FusedDense + tanh-GELU (8-wave core, VGPR accumulators) and x . W + r
    (4-wave core, AGPR accumulators)."""
    from gomlx_hip.backend import Backend, ActivationType, dtypes, make_shape
    monkeypatch.setenv("GHIP_RTC_DUMP", str(tmp_path))
    be = Backend("plan")
    b = be.Builder("dense")
    f = b.Main()
    x = f.Parameter("x", make_shape(dtypes.BFloat16, 8, 1024, 2048))
    if case == "gelu":
        w = f.Parameter("w", make_shape(dtypes.BFloat16, 2048, 8192))
        bias = f.Parameter("b", make_shape(dtypes.BFloat16, 8192))
        f.Return([f.FusedDense(x, w, bias, ActivationType.GELU)])
    else:
        w = f.Parameter("w", make_shape(dtypes.BFloat16, 2048, 2048))
        r = f.Parameter("r", make_shape(dtypes.BFloat16, 8, 1024, 2048))
        f.Return([f.Add(f.DotGeneral(x, [2], [], w, [0], []), r)])
    plan = b.Compile().Plan()
    assert ("core=8w-km32" if case == "gelu" else "core=4w-km32") in plan, plan
    srcs = [p for p in os.listdir(tmp_path) if p.startswith("gemm_epilogue") and p.endswith(".hip")]
    assert srcs, os.listdir(tmp_path)
    lines = _compile(str(tmp_path / srcs[0]), str(tmp_path / "epi.s"), ("-ffp-contract=off",))
    count, bad = _violations(lines, ["gemm_epilogue"])
    assert count >= 256, count
    assert not bad, bad[:5]
