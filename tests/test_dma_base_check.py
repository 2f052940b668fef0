"""The checker of aar-vlm_amd/check_dma_bases.py on small assembly texts (no
compiler, no GPU): a scalar-base DMA whose base comes from kernel arguments,
scalar arithmetic and SGPR spill restores passes; one whose base was written
by a VALU instruction, or moved to SGPRs by readfirstlane of a per-lane value,
fails; a kernel with DMAs and VGPR spills fails."""
from __future__ import annotations

import importlib.util
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def _checker():
    spec = importlib.util.spec_from_file_location("check_dma_bases", ROOT / "aar-vlm_amd" / "check_dma_bases.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _asm(body: str, spills: int = 0) -> str:
    return f"""kern:
{body}
\ts_endpgm
.Lfunc_end0:
amdhsa.kernels:
  - .name:           kern
    .private_segment_fixed_size: 0
    .vgpr_spill_count: {spills}
"""


GOOD = """\ts_load_dwordx4 s[4:7], s[0:1], 0x0
\ts_waitcnt lgkmcnt(0)
\ts_lshl_b32 s8, s2, 12
\ts_add_u32 s10, s4, s8
\ts_addc_u32 s11, s5, 0
\tv_readlane_b32 s12, v40, 3
\ts_add_u32 s10, s10, s12
\ts_mov_b32 m0, s9
\tglobal_load_lds_dwordx4 v2, s[10:11] offset:0"""


def test_scalar_chain_passes():
    origins, failures = _checker().check(_asm(GOOD))
    assert failures == []
    kinds = " ".join(origins)
    assert "kernel argument" in kinds and "spill restore" in kinds


def test_valu_written_base_fails():
    bad = GOOD.replace("\ts_add_u32 s10, s10, s12", "\tv_mov_b32 s10, v7")
    _, failures = _checker().check(_asm(bad))
    assert failures and "VALU" in failures[0]


def test_readfirstlane_of_a_lane_value_fails():
    bad = GOOD.replace("\ts_add_u32 s10, s10, s12", "\tv_add_u32 v9, v1, v3\n\tv_readfirstlane_b32 s10, v9")
    _, failures = _checker().check(_asm(bad))
    assert failures and "readfirstlane" in failures[0]


def test_readfirstlane_of_a_scalar_reciprocal_passes():
    ok = GOOD.replace("\ts_add_u32 s10, s10, s12", "\tv_cvt_u32_f32_e32 v9, v8\n\tv_readfirstlane_b32 s10, v9")
    origins, failures = _checker().check(_asm(ok))
    assert failures == []
    assert any("v_cvt_u32_f32" in k for k in origins)


def test_vgpr_spills_in_a_dma_kernel_fail():
    _, failures = _checker().check(_asm(GOOD, spills=4))
    assert failures and "spill" in failures[0]
