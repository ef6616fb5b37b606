"""bench.py's contract on a host without a GPU: more than one GPU is refused
with a message and exit status 2, before any device work."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in (r.stdout + r.stderr)
    assert r.stdout.strip() == "" or not r.stdout.lstrip().startswith("{")


def test_logit_buffer_note_says_when_the_logits_are_cache_resident():
    """A rotation whose buffers fit the 256 MB Infinity Cache is labelled
    cache-resident; one that exceeds it reads HBM."""
    import numpy as np

    sys.path.insert(0, ROOT)
    import bench

    small = bench.logit_buffers_note([np.zeros((1, 151_936), np.float32)] * 8)
    assert small["cache_resident"] and "cache-resident" in small["why"]
    assert small["bytes"] == 8 * 151_936 * 4
    big = bench.logit_buffers_note([np.zeros((64, 248_320), np.float32)] * 5)
    assert not big["cache_resident"] and "HBM" in big["why"]


def test_decode_parity_checks_every_step_against_the_oracle_loop():
    """bench's config-2 decode check: step i is the oracle's sample_logits on
    the prompt plus the first i drawn tokens with the i-th draw; feeding it
    the oracle's own loop gives no mismatch, and a changed token is caught at
    its step."""
    import numpy as np

    sys.path.insert(0, ROOT)
    import bench
    from lumen_amd.workloads import config2
    from oracle import oracle as o

    w = config2()
    op = bench.oracle_params(w)[0]
    rng = o.Xorshift64(w.seeds[0])
    hist = list(w.histories[0])
    drawn = []
    for _ in range(6):
        t = o.sample_logits_r(w.logits[0], op, np.asarray(hist, np.uint32), rng.next_f32())[0]
        drawn.append(t)
        hist.append(t)
    rep = bench.b1_decode_parity(drawn, 2)
    assert rep["mismatch"] == 0 and rep["steps"] == 6
    bad = list(drawn)
    bad[3] = (bad[3] + 1) % w.vocab
    rep = bench.b1_decode_parity(bad, 2)
    assert rep["first_mismatch_step"] == 3
