"""GEMM plan tables: a table saved by one process makes another run the same
plans and produce bit-identical parameters (the reference's determinism
goal, tests/hardware/test_determinism_fingerprint.py:88, across processes);
the table survives a text round trip; an imported plan that does not fit its
call's extents is re-planned, never launched."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

CHILD = r"""
import sys
import numpy as np
sys.path[:0] = [{root!r}, {pkg!r}]
from ttrl_amd.engine.device import open_device
from tests._dqn_helpers import build_learner
from ttrl_amd.workloads import dqn_batch
dev = open_device(0)
learner, _, _ = build_learner(dev, seed=7)
for k in range(3):
    learner.update(dqn_batch(70 + k))
np.savez({out!r}, **learner.online.state_dict())
dev.save_plans({plans!r})
learner.close()
print("child done", flush=True)
"""


def _child(tmp: Path, name: str, plans_in: str) -> dict:
    out, plans = tmp / f"{name}.npz", tmp / f"{name}.tsv"
    code = CHILD.format(root=str(ROOT), pkg=str(ROOT / "tt-rl_amd"), out=str(out), plans=str(plans))
    env = dict(os.environ, TTRL_PLANS=plans_in)
    proc = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=240)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    with np.load(out) as f:
        return {k: f[k] for k in f.files}, plans.read_text()


def test_a_saved_table_makes_a_second_process_agree_bit_for_bit(tmp_path):
    first, table = _child(tmp_path, "first", "none")  # tunes every signature itself
    assert len(table.splitlines()) >= 8
    second, table2 = _child(tmp_path, "second", str(tmp_path / "first.tsv"))
    assert table2 == table  # nothing re-tuned: every signature came from the file
    for k in first:
        assert np.array_equal(first[k], second[k]), k


def test_plan_table_text_round_trip_and_invalid_plans(device, monkeypatch):
    from ttrl_amd.engine.device import Device
    from ttrl_amd.workloads import dqn_batch
    from tests._dqn_helpers import build_learner

    monkeypatch.setenv("TTRL_PLANS", "none")  # contexts below start with empty tables
    clean = Device(0)
    try:
        learner, _, _ = build_learner(clean, seed=8)
        learner.update(dqn_batch(80))
        learner.close()
        text = clean.export_plans()
    finally:
        clean.close()
    lines = [ln for ln in text.splitlines() if ln]
    assert lines and all("\t" in ln for ln in lines)
    used = {ln.split("\t", 1)[1] for ln in lines}  # the signatures one DQN update calls
    other = Device(0)
    try:
        assert other.import_plans(text) == len(lines)
        assert other.export_plans() == text
        # every plan made to cover the wrong K range: each must be rejected and re-planned
        bad = "\n".join("0 32 32 256 9 256\t" + k for k in sorted(used)) + "\n"
        other.import_plans(bad)
        lr, _, _ = build_learner(other, seed=8)
        m = lr.update(dqn_batch(80))
        lr.close()
        assert np.isfinite(m["loss"])
        fixed = {ln.split("\t", 1)[1]: ln.split("\t", 1)[0] for ln in other.export_plans().splitlines() if ln}
        assert all(fixed[k] != "0 32 32 256 9 256" for k in used)
    finally:
        other.close()


CHILD_UPDATES = r"""
import sys
sys.path[:0] = [{root!r}, {pkg!r}]
from ttrl_amd.engine.device import open_device
from tests._dqn_helpers import build_learner
from tests._sac_helpers import build_sac
from ttrl_amd.workloads import dqn_batch, sac_batch
dev = open_device(0)
dqn, _, _ = build_learner(dev, seed=1)
dqn.update(dqn_batch(1))
sac, _, _ = build_sac(dev, seed=1)
sac.update(sac_batch(1))
sac.update(sac_batch(2))
dev.save_plans({plans!r})
print("child done", flush=True)
"""


def test_the_learner_updates_find_every_plan_in_the_packaged_table(tmp_path):
    """The DQN update at batch 32 and the SAC update at batch 256 (graph
    mode, the learners' defaults) call no GEMM signature the packaged table
    lacks: no process times candidates and picks plans of its own, so every
    process sums split partials in the same order."""
    packaged = ROOT / "tt-rl_amd" / "ttrl_amd" / "plans" / "gfx950.tsv"
    plans = tmp_path / "after.tsv"
    code = CHILD_UPDATES.format(root=str(ROOT), pkg=str(ROOT / "tt-rl_amd"), plans=str(plans))
    env = {k: v for k, v in os.environ.items() if k != "TTRL_PLANS"}  # the packaged table
    proc = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=240)
    assert proc.returncode == 0, proc.stdout + proc.stderr

    def entries(text):
        return {line.split("\t", 1)[1]: line.split("\t", 1)[0] for line in text.splitlines() if "\t" in line}

    before, after = entries(packaged.read_text()), entries(plans.read_text())
    extra = sorted(set(after) - set(before))
    assert not extra, "signatures missing from the packaged table:\n" + "\n".join(k[-120:] for k in extra)
    assert all(after[k] == before[k] for k in after)
