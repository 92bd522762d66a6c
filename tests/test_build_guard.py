"""The build refuses kernels that fall back to scratch memory or spill (no GPU needed)."""

from __future__ import annotations

import pytest

from kernelforge import build


def test_resource_guard_rejects_scratch_and_spills():
    ok = """x.hip:1:1: remark: Function Name: k_ok [-Rpass-analysis=kernel-resource-usage]
x.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:1:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]"""
    build._check_resources(ok, "x.hip")
    bad = ok + """
x.hip:9:1: remark: Function Name: k_bad [-Rpass-analysis=kernel-resource-usage]
x.hip:9:1: remark:     ScratchSize [bytes/lane]: 576 [-Rpass-analysis=kernel-resource-usage]"""
    with pytest.raises(RuntimeError, match="k_bad: ScratchSize"):
        build._check_resources(bad, "x.hip")
    spill = ok.replace("VGPRs Spill: 0", "VGPRs Spill: 12")
    with pytest.raises(RuntimeError, match="k_ok: VGPRs Spill = 12"):
        build._check_resources(spill, "x.hip")


def test_dma_wait_all_switch(monkeypatch):
    """KF_DMA_WAIT_ALL=1 adds the define that turns every counted LDS-DMA wait into vmcnt(0)."""
    monkeypatch.delenv("KF_DMA_WAIT_ALL", raising=False)
    assert "-DKF_DMA_WAIT_ALL" not in build.device_flags()
    monkeypatch.setenv("KF_DMA_WAIT_ALL", "1")
    assert "-DKF_DMA_WAIT_ALL" in build.device_flags()
    monkeypatch.setenv("KF_DMA_WAIT_ALL", "0")
    assert "-DKF_DMA_WAIT_ALL" not in build.device_flags()
