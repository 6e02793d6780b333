"""Host-side logic that needs no GPU: bench.py's one-GPU contract and the
decode model's attention-window buckets."""
import os
import subprocess
import sys
import types

import pytest

from zlm_amd.decode import DecodeModel

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("gpus", [2, 8])
def test_bench_refuses_more_than_one_gpu(gpus):
    """bench.py measures one GPU; --gpus N > 1 exits 2 with a message before
    touching a device."""
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", str(gpus)], cwd=ROOT,
                       capture_output=True, text=True, timeout=120)
    assert p.returncode == 2, p.stderr
    assert f"--gpus {gpus} is not supported" in p.stderr
    assert p.stdout == ""  # no JSON line


def _window(max_seq, pos):
    return DecodeModel.window_for(types.SimpleNamespace(cfg=types.SimpleNamespace(max_seq=max_seq)), pos)


@pytest.mark.parametrize("max_seq", [128, 2048, 3000, 32768])
def test_window_buckets(max_seq):
    """The window a step at `pos` replays: the smallest power of two >= pos + 1
    (at least 128), capped at max_seq; so a step never reads past its window
    and at most doubles the positions it needs."""
    seen = set()
    for pos in range(max_seq):
        w = _window(max_seq, pos)
        seen.add(w)
        assert pos < w <= max_seq
        if w < max_seq:
            assert w >= 128 and w & (w - 1) == 0
            assert w == 128 or w // 2 < pos + 1
    # one graph per bucket: the powers of two from 128 below max_seq, and max_seq itself
    want = {max_seq}
    b = 128
    while b < max_seq:
        want.add(b)
        b *= 2
    assert seen == want
