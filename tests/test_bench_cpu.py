"""bench.py's host-side pieces that need no GPU: the traffic table it reads
for roofline.traffic (profiles/attn_traffic.md) covers every kernel and
config the JSON line reports, and the multi-GPU refusal."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_traffic_table_covers_every_reported_config():
    t = bench.load_traffic()
    for cfg in ("c2", "c3", "c5"):
        for kern in ("attn_fwd", "attn_bwd_prepass", "attn_bwd_dkdv", "attn_bwd_dq"):
            assert (cfg, kern) in t, (cfg, kern)
            assert t[(cfg, kern)] > 0
    # HBM bytes at least the algorithmic minimum (each tensor once) and within
    # 1.5x of it.  c2's backward goes through the stored dS: dK/dV writes it
    # (B*H x S rounded up to 32 x S rounded up to 256, bf16), dQ reads it with
    # K and writes dQ.
    B, S, H, D = 1, 4608, 24, 128
    tensor, row = B * S * H * D * 2, B * H * S * 4
    ds = B * H * ((S + 31) // 32 * 32) * ((S + 255) // 256 * 256) * 2
    alg = {"attn_fwd": 4 * tensor + row, "attn_bwd_dkdv": 6 * tensor + 2 * row + ds, "attn_bwd_dq": 2 * tensor + ds}
    for kern, minimum in alg.items():
        assert minimum <= t[("c2", kern)] <= 1.5 * minimum, kern


def test_traffic_table_missing_gives_none(tmp_path):
    assert bench.load_traffic(str(tmp_path / "absent.md")) == {}


def test_multi_gpu_request_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "single-GPU" in r.stderr
