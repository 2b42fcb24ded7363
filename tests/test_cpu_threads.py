"""configure_flashlog_cpu_threads (flashlog_kernel.py:13-102): the "auto"
tiers for known machine shapes, and the FLASHLOG_CPU_THREADS /
FLASHLOG_CPU_INTEROP_THREADS switches applied to torch's pools."""
import pytest
import torch

from flashlog_amd.flashlog_kernel import flashlog_kernel as fk


# (logical CPUs, physical cores or None, threads): the reference's rule worked
# by hand -- 96+ CPUs: half the usable cores in [16, 32]; 48+: half in
# [12, 24]; 24+: the usable cores in [8, 16]; fewer: every logical CPU; no
# core count: half the logical CPUs from 8 up.
AUTO = [(192, 96, 32), (96, 48, 24), (96, None, 24), (100, 10, 16), (128, 128, 32),
        (64, 32, 16), (48, 24, 12), (48, 96, 24), (60, None, 15),
        (32, 16, 16), (24, 12, 12), (24, None, 12), (30, 30, 16), (24, 4, 8),
        (16, 8, 16), (8, None, 8), (4, 2, 4), (1, None, 1)]


@pytest.mark.parametrize("logical,physical,want", AUTO)
def test_auto_tiers(logical, physical, want):
    assert fk._auto_cpu_threads(logical, physical) == want


def test_machine_cores_is_sane():
    cores = fk._machine_cores()
    assert cores is None or 1 <= cores <= 4096


@pytest.fixture
def restore_threads():
    before = torch.get_num_threads()
    yield
    torch.set_num_threads(before)
    fk._FLASHLOG_CPU_THREADS_CONFIGURED = False


def test_switches(monkeypatch, restore_threads):
    logical = fk._logical_cpus()
    torch.set_num_threads(1)
    monkeypatch.setenv("FLASHLOG_CPU_THREADS", "off")
    assert fk.configure_flashlog_cpu_threads(force=True) == 1
    monkeypatch.setenv("FLASHLOG_CPU_THREADS", "2")
    assert fk.configure_flashlog_cpu_threads(force=True) == min(2, logical)
    monkeypatch.setenv("FLASHLOG_CPU_THREADS", "3")
    # configured once: without force the setting is not read again
    assert fk.configure_flashlog_cpu_threads() == min(2, logical)
    monkeypatch.setenv("FLASHLOG_CPU_THREADS", "-4")
    assert fk.configure_flashlog_cpu_threads(force=True) == 1
    monkeypatch.setenv("FLASHLOG_CPU_THREADS", "100000")
    assert fk.configure_flashlog_cpu_threads(force=True) == logical
    for auto in ("auto", "", "many"):
        monkeypatch.setenv("FLASHLOG_CPU_THREADS", auto)
        assert fk.configure_flashlog_cpu_threads(force=True) == min(fk._auto_cpu_threads(), logical)
    monkeypatch.delenv("FLASHLOG_CPU_THREADS")
    torch.set_num_threads(1)
    assert fk.configure_flashlog_cpu_threads(force=True) == 1  # unset means "off"
    monkeypatch.setenv("FLASHLOG_CPU_INTEROP_THREADS", "not a number")
    monkeypatch.setenv("FLASHLOG_CPU_THREADS", "1")
    assert fk.configure_flashlog_cpu_threads(force=True) == 1
