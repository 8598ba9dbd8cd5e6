"""The kernels' inline asm carries the wait states the compiler would have inserted.

The compiler guards hardware hazards only between instructions it generated;
``csrc/asm_hazards.py`` checks every inline-asm VMEM / VALU instruction of the
gfx950 assembly of this build (``make asm``) against the hazards that can reach one
here (a VALU-written SGPR read by a buffer load within 5 wait states, an MFMA result
read by a VALU within 8, a transcendental result read by a VALU within 1).  The checker itself is pinned on planted cases."""
import importlib.util
import os
import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "adaptive-kv-memory_amd" / "csrc"


def _checker():
    spec = importlib.util.spec_from_file_location("asm_hazards", CSRC / "asm_hazards.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


_MFMA_THEN_ASM = """
k:
	v_mfma_f32_16x16x32_f16 v[72:75], v[118:121], v[64:67], v[72:75]
	s_cbranch_scc1 .LBB0_2
	v_cndmask_b32_e32 v72, v115, v72, vcc
.LBB0_2:
	;;#ASMSTART
	v_max3_f32 v77, v71, v72, v73
	;;#ASMEND
"""

_READLANE_THEN_DMA = """
k:
	v_readlane_b32 s74, v164, 33
	v_readlane_b32 s75, v164, 34
	;;#ASMSTART
	s_mov_b32 s5, m0
	s_mov_b32 m0, s3
	s_nop {nop}
	buffer_load_dwordx4 v94, s[72:75], s2 offen offset:0 nt lds
	s_mov_b32 m0, s5
	;;#ASMEND
"""


def test_checker_finds_planted_hazards():
    chk = _checker()
    # the MFMA reaches the asm max on both paths: through the branch (1 wait state) and
    # through the fall-through (2: the cndmask rewrote v72, but v73 is still the MFMA's)
    n, hz = chk.check(_MFMA_THEN_ASM)
    assert n == 1 and len(hz) == 2 and all("MFMA" in h for h in hz)
    assert "1 wait states" in hz[0] + hz[1] and "2 wait states" in hz[0] + hz[1]
    # the fall-through path alone
    n, hz = chk.check(_MFMA_THEN_ASM.replace("s_cbranch_scc1 .LBB0_2\n", ""))
    assert n == 1 and len(hz) == 1
    # enough s_nop before the read: none
    n, hz = chk.check(_MFMA_THEN_ASM.replace("s_cbranch_scc1 .LBB0_2\n", "s_nop 7\n"))
    assert n == 1 and hz == []
    # descriptor words reloaded by v_readlane 3 and 4 wait states before the load
    n, hz = chk.check(_READLANE_THEN_DMA.format(nop=0))
    assert n == 1 and len(hz) == 2 and all("SGPR" in h for h in hz)
    # s_nop 2 makes 5 and 6
    n, hz = chk.check(_READLANE_THEN_DMA.format(nop=2))
    assert n == 1 and hz == []
    # a reciprocal read by the next (asm) instruction, then with one instruction between
    rcp = "k:\n\tv_rcp_f32_e32 v3, v2\n{mid}\t;;#ASMSTART\n\tv_fma_mixlo_f16 v5, v4, v3, 0\n\t;;#ASMEND\n"
    n, hz = chk.check(rcp.format(mid=""))
    assert n == 1 and len(hz) == 1 and "transcendental" in hz[0]
    n, hz = chk.check(rcp.format(mid="\tv_mov_b32_e32 v6, v7\n"))
    assert n == 1 and hz == []


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc is not installed")
def test_kernel_inline_asm_has_its_wait_states(tmp_path):
    subprocess.run(["make", "-s", "-C", str(CSRC), "-j8", "asm", f"ASMDIR={tmp_path}"], check=True,
                   stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    chk = _checker()
    total = 0
    for s in sorted(tmp_path.glob("*.s")):
        n, hz = chk.check(s.read_text())
        assert hz == [], f"{s.name}: " + "\n".join(hz[:10])
        total += n
    # the LDS-DMA loads of the decode kernels and the dequant helpers are in asm
    assert total > 1000
