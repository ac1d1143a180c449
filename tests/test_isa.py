"""Static check of the panel kernel's gfx950 code for a hazard the compiler
cannot see: its steps are inline assembly with DPP operands (v_add_u32_dpp,
v_fmac_f32_dpp row_newbcast), and on gfx9 a DPP instruction that reads a VGPR
written by a VALU instruction needs two wait states between the two.  The
compiler inserts these for its own DPP instructions but does not look inside
inline assembly, so this test compiles the library's device code to assembly
and walks back from every DPP instruction along every path (fall-through and
branches into its block) to the second wait state."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")

_INSTR = re.compile(r"^\s+([a-z_][a-z0-9_]*)(\s+(.*))?$")
_LABEL = re.compile(r"^(\.?[A-Za-z_$][\w.$]*):")
_VREG = re.compile(r"^v(\d+)$|^v\[(\d+):(\d+)\]$")


def regs(op):
    m = _VREG.match(op.strip())
    if not m:
        return set()
    if m.group(1) is not None:
        return {int(m.group(1))}
    return set(range(int(m.group(2)), int(m.group(3)) + 1))


def parse(lines):
    """[(kind, payload)] with kind 'label' (name) or 'instr' (mnemonic, operands)."""
    out = []
    for ln in lines:
        code = ln.split(";")[0].rstrip()
        if not code.strip():
            continue
        m = _LABEL.match(code)
        if m:
            out.append(("label", m.group(1)))
            continue
        m = _INSTR.match(code)
        if m and not m.group(1).startswith("."):
            ops = [o.strip() for o in (m.group(3) or "").split(",")]
            out.append(("instr", (m.group(1), ops)))
    return out


def dpp_hazards(body):
    """DPP instructions whose DPP source (src0) a VALU instruction writes less
    than two wait states before, on some path."""
    prog = parse(body)
    branches = {}  # label -> indices of branch instructions to it
    for i, (kind, x) in enumerate(prog):
        if kind == "instr" and x[0].startswith(("s_cbranch", "s_branch")):
            branches.setdefault(x[1][0], []).append(i)
    bad = []

    def walk(i, src, budget, seen):
        # instructions before index i (exclusive) on every path into i
        while i > 0:
            i -= 1
            kind, x = prog[i]
            if kind == "label":
                for b in branches.get(x, []):
                    if (b, budget) not in seen:
                        seen.add((b, budget))
                        if walk(b + 1, src, budget, seen):
                            return True
                continue
            mn, ops = x
            if mn in ("s_branch", "s_endpgm", "s_setpc_b64"):
                return False  # no fall-through into what follows
            if mn.startswith("v_") and ops and regs(ops[0]) & src and not mn.startswith(("v_readlane", "v_readfirstlane", "v_cmp")):
                return True
            budget -= int(ops[0]) + 1 if mn == "s_nop" else 1
            if budget <= 0:
                return False
        return False

    for i, (kind, x) in enumerate(prog):
        if kind != "instr" or not x[0].endswith("_dpp"):
            continue
        src = regs(x[1][1]) if len(x[1]) > 1 else set()
        if src and walk(i, src, 2, set()):
            bad.append((i, x))
    return bad


@pytest.fixture(scope="module")
def device_asm(tmp_path_factory):
    out = tmp_path_factory.mktemp("isa") / "tca_spmm.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", "-o", str(out), "-I" + os.path.join(ROOT, "include"),
           os.path.join(ROOT, "spmm_amd", "csrc", "tca_spmm.hip")]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text().splitlines()


def functions(lines, pattern):
    out, cur = {}, None
    for ln in lines:
        m = re.match(r"^(_Z\w+):", ln)
        if m:
            cur = m.group(1) if pattern in m.group(1) else None
            if cur:
                out[cur] = []
            continue
        if cur is not None:
            out[cur].append(ln)
            if "s_endpgm" in ln:
                cur = None
    return out


def test_walker_finds_a_planted_hazard():
    body = ["\tv_lshl_add_u32 v5, v1, 9, v2", "\tv_add_u32_dpp v6, v5, v3 row_newbcast:0 row_mask:0xf bank_mask:0xf"]
    assert dpp_hazards(body)
    assert not dpp_hazards([body[0], "\ts_nop 1", body[1]])
    # through a branch into the DPP instruction's block
    body = ["\tv_mov_b32_e32 v5, v1", "\ts_cbranch_scc1 .LBB0_2", "\ts_nop 4", ".LBB0_2:",
            "\tv_fmac_f32_dpp v7, v5, v3 row_newbcast:1 row_mask:0xf bank_mask:0xf"]
    assert dpp_hazards(body)
    assert not dpp_hazards(["\tv_mov_b32_e32 v9, v1", "\tv_fmac_f32_dpp v7, v5, v3 row_newbcast:1"])


def test_panel_kernel_dpp_wait_states(device_asm):
    fns = functions(device_asm, "panel_kernel")
    assert len(fns) >= 7, sorted(fns)
    n_dpp = 0
    for name, body in fns.items():
        n_dpp += sum("_dpp " in ln for ln in body)
        bad = dpp_hazards(body)
        assert not bad, (name, bad[:5])
    assert n_dpp > 100
