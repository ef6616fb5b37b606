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


def _csr(params, hists):
    """Form B: each row's (distinct id, count) window as device tensors."""
    import torch

    offs, ids, cnts = [0], [], []
    for p, h in zip(params, hists):
        h = np.asarray(h, np.uint32)
        if p.penalties_active() and h.size:
            u, c = np.unique(h, return_counts=True)
            ids.append(u)
            cnts.append(c.astype(np.uint32))
            offs.append(offs[-1] + u.size)
        else:
            offs.append(offs[-1])
    cat = lambda xs: np.concatenate(xs).astype(np.uint32) if xs else np.zeros(1, np.uint32)
    t = lambda a: torch.from_numpy(np.asarray(a, np.uint32).view(np.int32)).cuda()
    return t(np.array(offs, np.uint32)), t(cat(ids)), t(cat(cnts))


def test_noalloc_allocates_nothing_and_replays_under_capture():
    """A noalloc call of a new shape leaves the device's free memory
    unchanged; captured into a HIP graph (device penalty counts, inline rows,
    device draws) every replay matches the eager lumen_sampler_sample_batch
    result, with eager noalloc calls on other inputs between the replays; a
    form-A history under capture is refused."""
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    eng = Engine(0)
    try:
        la, pa, ha, ua = _case(21, 8, 248_320)
        lb, pb, hb, ub = _case(22, 5, 151_936)
        dev_a, dev_b = torch.from_numpy(la).cuda(), torch.from_numpy(lb).cuda()
        csr_a, csr_b = _csr(pa, ha), _csr(pb, hb)
        ud_a, ud_b = torch.from_numpy(ua).cuda(), torch.from_numpy(ub).cuda()
        tok_a = torch.full((8,), -1, dtype=torch.int32, device="cuda")
        tok_b = torch.full((5,), -1, dtype=torch.int32, device="cuda")
        tok_g = torch.full((5,), -1, dtype=torch.int32, device="cuda")
        # warm-up on another shape, then the measured call
        eng.sample_batch(dev_a, pa, penalty_counts=csr_a, uniforms_dev=ud_a, tokens_out=tok_a,
                         sync=False, noalloc=True)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        eng.sample_batch(dev_b, pb, penalty_counts=csr_b, uniforms_dev=ud_b, tokens_out=tok_b,
                         sync=False, noalloc=True)
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0, "a noalloc call allocated device memory"
        got_b = tok_b.cpu().tolist()
        # the reference: the allocating entry point on the same inputs
        ref = torch.full((5,), -1, dtype=torch.int32, device="cuda")
        eng.sample_batch(dev_b, pb, penalty_counts=csr_b, uniforms_dev=ud_b, tokens_out=ref,
                         sync=False)
        ref_a = torch.full((8,), -1, dtype=torch.int32, device="cuda")
        eng.sample_batch(dev_a, pa, penalty_counts=csr_a, uniforms_dev=ud_a, tokens_out=ref_a,
                         sync=False)
        torch.cuda.synchronize()
        want_b, want_a = ref.cpu().tolist(), ref_a.cpu().tolist()
        assert got_b == want_b
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            eng.sample_batch(dev_b, pb, penalty_counts=csr_b, uniforms_dev=ud_b, tokens_out=tok_g,
                             sync=False, noalloc=True)
        for rep in range(4):
            tok_g.fill_(-1)
            tok_a.fill_(-1)
            # eager work on the same scratch array between replays
            eng.sample_batch(dev_a, pa, penalty_counts=csr_a, uniforms_dev=ud_a,
                             tokens_out=tok_a, sync=False, noalloc=True)
            torch.cuda.synchronize()
            assert tok_a.cpu().tolist() == want_a, rep
            g.replay()
            torch.cuda.synchronize()
            assert tok_g.cpu().tolist() == want_b, rep
        # form A needs a host copy: refused under capture, nothing recorded
        g2 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g2):
            with pytest.raises(RuntimeError):
                eng.sample_batch(dev_b, pb, histories=hb, uniforms_dev=ud_b, tokens_out=tok_g,
                                 sync=False, noalloc=True)
            tok_g.fill_(7)
        assert b"stream capture" in _native.load().lumen_sampler_last_error()
        g2.replay()
        torch.cuda.synchronize()
        assert tok_g.cpu().tolist() == [7] * 5
    finally:
        eng.close()
