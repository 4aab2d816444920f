"""CPU-only policy tests, restating the reference's tests/test_plan.py:9-16, 39-45
(the RDNA4 tile-picker known answers, test_plan.py:19-36, are tuning facts of the
reference's Triton kernels and have no counterpart here)."""
import os
import subprocess
import sys
from pathlib import Path

from rdna4_conv3d.conv3d_wmma import _geom_ok, conv3d_plan

ROOT = Path(__file__).resolve().parents[1]


def test_geom_ok_k1_k3_only():
    assert _geom_ok(3, 1, 1, 1)
    assert _geom_ok(1, 1, 1, 1)
    assert _geom_ok((3, 3, 3), (1, 1, 1), (1, 1, 1), 1)
    assert not _geom_ok(5, 1, 1, 1)
    assert not _geom_ok(3, 2, 1, 1)
    assert not _geom_ok(3, 1, 2, 1)
    assert not _geom_ok(3, 1, 1, 2)
    assert not _geom_ok((3, 3, 1), 1, 1, 1)
    assert not _geom_ok(2, 1, 1, 1)


def test_plan_values_are_wmma_or_miopen():
    plan = conv3d_plan(24, 24, 3)
    assert set(plan) == {"fwd", "dw", "dx"}
    assert plan["fwd"] in ("wmma", "miopen")
    slow = conv3d_plan(24, 24, 3, stride=2)
    assert slow == {"fwd": "miopen", "dw": "miopen", "dx": "miopen"}
    assert conv3d_plan(24, 24, 3, groups=2) == slow
    assert conv3d_plan(24, 24, 5) == slow


def _plan_in_subprocess(env_extra):
    env = dict(os.environ)
    env.pop("RDNA4_CONV3D_BACKEND", None)
    env.pop("BIOHUB_CONV3D_BACKEND", None)
    env.update(env_extra)
    code = ("import sys; sys.path.insert(0, %r); from rdna4_conv3d import conv3d_plan; "
            "print(conv3d_plan(24, 24, 3)['fwd'], conv3d_plan(24, 24, 3, stride=2)['fwd'])"
            % str(ROOT / "rdna4-conv3d-wmma_amd"))
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, check=True)
    return out.stdout.split()


def test_backend_env_selects_path():
    # wmma forces the native path for supported geometry; miopen / torch force the stock path.
    assert _plan_in_subprocess({"RDNA4_CONV3D_BACKEND": "wmma"}) == ["wmma", "miopen"]
    assert _plan_in_subprocess({"RDNA4_CONV3D_BACKEND": "miopen"}) == ["miopen", "miopen"]
    assert _plan_in_subprocess({"RDNA4_CONV3D_BACKEND": "torch"}) == ["miopen", "miopen"]
    # alias, and case-insensitive
    assert _plan_in_subprocess({"BIOHUB_CONV3D_BACKEND": "WMMA"}) == ["wmma", "miopen"]
    # hybrid without a gfx950 GPU: stock path
    import torch
    if not torch.cuda.is_available():
        assert _plan_in_subprocess({})[0] == "miopen"
