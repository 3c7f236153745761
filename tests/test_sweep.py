"""CPU tests of the tile-sweep tool (inkling_fa4.sweep): grid expansion, and
that a knob given at build time reaches the variant library a child process
loads through IFA4_LIB_DIR (checked with a host-only tile query)."""
import json
import os
import subprocess
import sys

import pytest

from inkling_fa4 import sweep

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(sweep.__file__)))


def test_grid_points_is_the_cartesian_product():
    pts = sweep._grid_points(["IFA4_LOOK_K=2,4", "IFA4_PRIO=0,1", "IFA4_SCHED=1"])
    assert len(pts) == 4
    assert {"IFA4_LOOK_K": "2", "IFA4_PRIO": "1", "IFA4_SCHED": "1"} in pts
    assert all(p["IFA4_SCHED"] == "1" for p in pts)


@pytest.mark.parametrize("bad", ["IFA4_LOOK_K", "=1,2", "IFA4_LOOK_K="])
def test_grid_rejects_malformed_specs(bad):
    with pytest.raises(SystemExit):
        sweep._grid_points([bad])


_TILE_QUERY = r"""
import ctypes, json
from inkling_fa4 import _abi
a = _abi.make_args(batch=64, n_heads=8, kv_heads=2, head_dim=128, rel_extent=128,
    rel_width=128, max_seqlen_q=1, max_seqlen_k=16384, total_q=64, total_k=600000,
    q=1 << 20, k=2 << 20, v=3 << 20, rel=4 << 20, out=5 << 20, cu_seqlens_q=6 << 20,
    cu_seqlens_k=7 << 20, q_stride_t=1024, q_stride_h=128, k_stride_t=256, k_stride_h=128,
    v_stride_t=256, v_stride_h=128, rel_stride_t=0, rel_stride_h=128, out_stride_t=1024,
    out_stride_h=128, softmax_scale=1 / 128, qkv_dtype=_abi.IFA4_BF16,
    rel_dtype=_abi.IFA4_FP32, causal=0)
t = _abi.Ifa4Tile()
assert _abi.lib().ifa4_decode_tile(ctypes.byref(a), ctypes.byref(t)) == 0
print(json.dumps({"kv_chunk": t.kv_chunk, "lib": _abi.LIB_PATH}))
"""


def _tile(lib_dir=None):
    env = dict(os.environ)
    env.pop("IFA4_LIB_DIR", None)
    if lib_dir:
        env["IFA4_LIB_DIR"] = lib_dir
    out = subprocess.run([sys.executable, "-c", _TILE_QUERY], env=env, cwd=PKG_ROOT,
                         capture_output=True, text=True, check=True).stdout
    return json.loads(out.strip().splitlines()[-1])


def test_variant_build_carries_its_knob(tmp_path):
    sweep.main(["build", "--dir", str(tmp_path), "--grid", "IFA4_DECODE_WAVES=512",
                "--jobs", "3"])
    vdir = tmp_path / "decode_waves512"
    assert sorted(os.listdir(vdir)) == ["_ifa4_torch.so", "knobs.json", "libifa4.so",
                                        "source.txt"]
    assert len((vdir / "source.txt").read_text().strip()) == 12
    assert json.loads((vdir / "knobs.json").read_text()) == {"IFA4_DECODE_WAVES": "512"}
    steps = 64 * 2 * (16384 // 32)
    default, variant = _tile(), _tile(str(vdir))
    assert variant["lib"] == str(vdir / "libifa4.so")
    assert default["kv_chunk"] == 32 * -(-steps // 896)
    assert variant["kv_chunk"] == 32 * -(-steps // 512)
