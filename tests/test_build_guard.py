"""The build's resource guard (unifiedkv_amd/_build.py): kernels that issue global loads by
inline asm and wait for them with a hand-placed s_waitcnt must compile without scratch and
without spilled VGPRs, since a spill could move a load's destination register while the load
is still in flight. CPU only: the parse is checked on fixed remark text, then every guarded
source is compiled for gfx950 (device code only) and its remarks checked."""
from concurrent.futures import ThreadPoolExecutor

import pytest

from unifiedkv_amd import _build

REMARKS = """\
x.hip:10:1: remark: Function Name: _ZN3ukv20paged_prefill_kernelILi1ELi8ELb1EEEvNS_11PrefillArgsE [-Rpass-analysis=kernel-resource-usage]
   10 | __global__ void f() {
      | ^
x.hip:10:1: remark:     VGPRs: 255 [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     ScratchSize [bytes/lane]: 20 [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     SGPRs Spill: 68 [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark: Function Name: _ZN3ukv16snap_tile_kernelILi1ELi128ELb1ELi4EEEvNS_8SnapArgsE [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark:     SGPRs Spill: 15 [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark:     VGPRs Spill: 3 [-Rpass-analysis=kernel-resource-usage]
x.hip:30:1: remark: Function Name: _ZN3ukv19page16_split_kernelILi0ELi128ELb0EEEvNS_10DecodeArgsE [-Rpass-analysis=kernel-resource-usage]
x.hip:30:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:30:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:40:1: remark: Function Name: _ZN3ukv27paged_prefill_scalar_kernelILi1EEEvNS_11PrefillArgsE [-Rpass-analysis=kernel-resource-usage]
x.hip:40:1: remark:     ScratchSize [bytes/lane]: 64 [-Rpass-analysis=kernel-resource-usage]
x.hip:40:1: remark:     VGPRs Spill: 9 [-Rpass-analysis=kernel-resource-usage]
"""


def test_parse_and_verdicts_on_fixed_remarks():
    usage = _build.parse_resource_usage(REMARKS)
    assert len(usage) == 4
    pp = usage["_ZN3ukv20paged_prefill_kernelILi1ELi8ELb1EEEvNS_11PrefillArgsE"]
    assert pp["VGPRs"] == "255" and pp["ScratchSize [bytes/lane]"] == "20" and pp["SGPRs Spill"] == "68"
    bad = _build.resource_violations(usage)
    # scratch in the prefill instance and spilled VGPRs in the SnapKV tile are refused; the clean
    # decode instance passes; the scalar prefill issues no hand-managed loads and is not guarded
    assert len(bad) == 2
    assert bad[0].startswith("_ZN3ukv20paged_prefill_kernel") and "ScratchSize 20" in bad[0]
    assert bad[1].startswith("_ZN3ukv16snap_tile_kernel") and "VGPRs spilled 3" in bad[1]
    assert not _build.guarded("_ZN3ukv27paged_prefill_scalar_kernelILi1EEEvNS_11PrefillArgsE")
    assert _build.guarded("_ZN3ukv20paged_prefill_kernelILi0ELi8ELb0EEEvNS_11PrefillArgsE")
    assert not _build.guarded("_ZN3ukv22obs_rows_finish_kernelILi1EEEvNS_11PrefillArgsE")


def test_incomplete_remarks_are_refused():
    text = REMARKS.split("x.hip:20:1")[0].replace("ScratchSize", "Scratch")
    assert "incomplete" in _build.resource_violations(_build.parse_resource_usage(text))[0]


def test_guarded_sources_compile_without_spills_or_scratch():
    try:
        _build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    with ThreadPoolExecutor(len(_build.GUARDED_SOURCES)) as ex:
        usages = list(ex.map(_build.guarded_resource_usage, _build.GUARDED_SOURCES))
    seen = set()
    for src, usage in zip(_build.GUARDED_SOURCES, usages):
        assert _build.resource_violations(usage) == [], src
        for k in _build.GUARDED_KERNELS:
            if any(_build.guarded(n) and f"{len(k)}{k}" in n for n in usage):
                seen.add(k)
    assert seen == set(_build.GUARDED_KERNELS)
