"""lumen_sampler_sample_batch_noalloc against lumen_sampler_sample_batch,
through the C ABI: two calls in a row, the second with a smaller batch and
vocabulary, tokens and intermediate sums bit for bit (gpu)."""
import numpy as np
import pytest

from lumen_amd import _native
from lumen_amd.sampling import Engine, SamplingParams as SP

pytestmark = pytest.mark.gpu


def _case(seed, B, V):
    rng = np.random.default_rng(seed)
    logits = (rng.normal(0, 3, (B, V)) + rng.gumbel(0, 1, (B, V))).astype(np.float32)
    kinds = [SP(temperature=0.0), SP(temperature=1.0, top_k=50), SP(temperature=1.0, top_p=0.9),
             SP(temperature=0.6, top_k=100, top_p=0.95, repetition_penalty=1.05),
             SP(temperature=0.7, top_p=0.9, repetition_penalty=1.05),
             SP(temperature=0.9, min_p=0.05), SP(temperature=1.0),
             SP(temperature=0.0, repetition_penalty=1.3)]
    params = [kinds[(b + seed) % len(kinds)] for b in range(B)]
    hists = [rng.integers(0, V, int(rng.integers(0, 600))).astype(np.uint32) for _ in range(B)]
    uniforms = rng.random(B).astype(np.float32)
    return logits, params, hists, uniforms


def _run(eng, logits, params, hists, uniforms, noalloc):
    import torch

    B = logits.shape[0]
    dev = torch.from_numpy(logits).cuda()
    tok = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    trace = torch.zeros((B, 16), dtype=torch.int32, device="cuda")
    eng.sample_batch(dev, params, histories=hists, uniforms=uniforms, tokens_out=tok, trace=trace,
                     sync=False, noalloc=noalloc)
    torch.cuda.synchronize()
    return tok.cpu().numpy(), trace.cpu().numpy()


def test_noalloc_matches_sample_batch():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    eng = Engine(0)
    try:
        for seed, B, V in ((11, 8, 248_320), (12, 3, 4099), (13, 8, 151_936)):
            case = _case(seed, B, V)
            want_tok, want_tr = _run(eng, *case, noalloc=False)
            got_tok, got_tr = _run(eng, *case, noalloc=True)
            assert got_tok.tolist() == want_tok.tolist(), (seed, B, V)
            # every trace word: status, path-independent sums and counts
            for f in (0, 2, 3, 4, 5, 6, 8, 9, 10, 11, 12):
                assert got_tr[:, f].tolist() == want_tr[:, f].tolist(), (seed, B, V, f)
    finally:
        eng.close()


def test_noalloc_rejects_sizes_beyond_its_limits():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    eng = Engine(0)
    try:
        logits, params, hists, uniforms = _case(14, 9, 512)
        with pytest.raises(RuntimeError):
            eng.sample_batch(torch.from_numpy(logits).cuda(), params, uniforms=uniforms, sync=False,
                             noalloc=True)
        assert b"8 rows" in _native.load().lumen_sampler_last_error()
    finally:
        eng.close()
