"""Register budget of every kernel (CPU; no GPU needed).

Every HIP translation unit of libfa_hip.so is compiled for gfx950 with the product's flags and
``-Rpass-analysis=kernel-resource-usage``; the compiler then reports, per kernel, its VGPRs,
AGPRs, spills, scratch and occupancy. The budget (the static per-tile budgets of
ref:include/fa/tile_config.h:189-210, restated for gfx950's 256-VGPR waves):

* no kernel spills a VGPR or uses scratch memory: a spill puts scratch loads and a ``vmcnt`` wait
  into the key loop, and a variant that spilled was measured slower than every one that did not;
* the stage-5 default tiles keep the occupancy their launch geometry assumes: 8-wave workgroups
  need 2 waves per SIMD (one workgroup per CU); the narrow 4-wave tiles need 2 (two workgroups
  per CU) and the D = 64 narrow tile 3.
"""

from __future__ import annotations

import importlib.util
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "fused-attention-cuda_amd"

spec = importlib.util.spec_from_file_location("fa_build", PKG / "build.py")
fa_build = importlib.util.module_from_spec(spec)
spec.loader.exec_module(fa_build)

pytestmark = pytest.mark.skipif(not Path(fa_build.HIPCC).exists() and shutil.which("hipcc") is None,
                                reason="hipcc not found")

_NAME = re.compile(r"remark: Function Name: (\S+)")
_FIELD = re.compile(r"remark:\s+([A-Za-z][A-Za-z /]*?)(?: \[[^\]]*\])?: (\d+)")


def resource_report(source: str) -> dict[str, dict[str, int]]:
    """{mangled kernel name: {field: value}} from the compiler's resource-usage remarks."""
    cmd = [fa_build.HIPCC, *fa_build.HIP_FLAGS, "--cuda-device-only", "-c", "-o", "/dev/null",
           str(fa_build.CSRC / source), "-Rpass-analysis=kernel-resource-usage"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    report: dict[str, dict[str, int]] = {}
    current = None
    for line in res.stderr.splitlines():
        if m := _NAME.search(line):
            current = report.setdefault(m.group(1), {})
        elif current is not None and (m := _FIELD.search(line)):
            current[m.group(1).strip()] = int(m.group(2))
    return report


@pytest.fixture(scope="module")
def kernels() -> dict[str, dict[str, int]]:
    with ThreadPoolExecutor(max_workers=len(fa_build.HIP_SOURCES)) as pool:
        reports = list(pool.map(resource_report, fa_build.HIP_SOURCES))
    merged = {name: fields for r in reports for name, fields in r.items()}
    assert merged, "the compiler reported no kernels"
    return merged


def test_every_kernel_is_spill_and_scratch_free(kernels):
    bad = {name: (f.get("VGPRs Spill"), f.get("ScratchSize")) for name, f in kernels.items()
           if f.get("VGPRs Spill", 0) or f.get("ScratchSize", 0)}
    assert not bad, f"kernels that spill or use scratch (VGPR spills, scratch bytes): {bad}"


def test_every_kernel_was_reported(kernels):
    families = {"fa_s5_tuned", "fa_s4_mfma", "fa_s3_fused", "fa_s5_combine", "fa_decode_split",
                "fa_decode_combine"}
    seen = {fam for fam in families for name in kernels if fam in name}
    assert seen == families, f"missing from the report: {families - seen}"
    # Two dtypes x (12 D=64 + 8 D=128) stage-5 tiles.
    assert sum("fa_s5_tuned" in name for name in kernels) == 40


# (dtype tag in the mangled name, D, RG, KS, BCW) -> occupancy (waves per SIMD) the launch
# geometry needs.
_OCCUPANCY = {
    ("DF16_", 64, 4, 2, 64): 2,   # D = 64 default: BR 128 / BC 128, 8 waves, one per CU
    ("DF16_", 128, 4, 2, 32): 2,  # D = 128 default: BR 128 / BC 64, 8 waves
    ("DF16_", 64, 2, 2, 32): 3,   # D = 64 narrow: BR 64 / BC 64, 4 waves, three per CU
    ("DF16_", 128, 4, 1, 32): 2,  # D = 128 narrow: BR 128 / BC 32, 4 waves, two per CU
    ("DF16b", 128, 4, 1, 32): 2,  # the same for bf16 (LONG)
    ("DF16b", 128, 4, 2, 32): 2,
}


@pytest.mark.parametrize("key", list(_OCCUPANCY), ids=lambda k: "%s-D%d-%d-%d-%d" % k)
def test_default_tiles_keep_their_occupancy(kernels, key):
    tag, d, rg, ks, bcw = key
    name = f"_ZN2fa3m1611fa_s5_tunedI{tag}Li{d}ELi{rg}ELi{ks}ELi{bcw}EEEvNS_5KArgsE"
    assert name in kernels, name
    assert kernels[name]["Occupancy"] >= _OCCUPANCY[key], kernels[name]
