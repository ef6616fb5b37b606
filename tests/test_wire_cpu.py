"""Request-level parameters (lumen_amd.wire) against the server wire layer's
rules: crates/lumen-server/src/wire/openai.rs:184-243, 357-381,
wire/mod.rs:81-220 and runtime_defaults.rs:431-521, 970-999. The expected
values are the reference's own test expectations where it has them
(normalize_zero_penalty_matches_cli, next_random_seed_unique_across_threads,
repeat_last_n_resolved_env_precedence) and its documented defaults otherwise.
"""
import threading

import pytest

from lumen_amd import wire
from lumen_amd.wire import ModelHint


@pytest.fixture(autouse=True)
def clean_env(monkeypatch):
    for k in ("LUMEN_REPETITION_PENALTY", "LUMEN_FREQUENCY_PENALTY", "LUMEN_REPEAT_LAST_N",
              "LUMEN_ANTI_RESTATE"):
        monkeypatch.delenv(k, raising=False)


def test_normalize_zero_penalty_matches_cli():
    # wire/mod.rs:261-290
    assert wire.normalize_zero_penalty(None) is None
    assert wire.normalize_zero_penalty(0.0) is None
    assert wire.normalize_zero_penalty(-0.0) is None
    assert wire.normalize_zero_penalty(float("nan")) is None
    assert wire.normalize_zero_penalty(float("inf")) is None
    assert wire.normalize_zero_penalty(0.7) == pytest.approx(0.7)


def test_next_random_seed_unique_across_threads():
    # wire/mod.rs:228-245 (8 threads x 20k draws, no duplicate)
    out = [[] for _ in range(8)]

    def run(i):
        out[i] = [wire.next_random_seed() for _ in range(20000)]

    ts = [threading.Thread(target=run, args=(i,)) for i in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    seen = set()
    for o in out:
        seen.update(o)
    assert len(seen) == 8 * 20000


def test_repeat_last_n_env_precedence(monkeypatch):
    # runtime_defaults.rs:2759-2780
    assert wire.repeat_last_n_resolved() is None
    monkeypatch.setenv("LUMEN_REPEAT_LAST_N", "64")
    assert wire.repeat_last_n_resolved() == 64
    monkeypatch.setenv("LUMEN_REPEAT_LAST_N", "0")
    assert wire.repeat_last_n_resolved() == 0
    for bad in ("-1", "12.5", "garbage", "", " 64"):
        monkeypatch.setenv("LUMEN_REPEAT_LAST_N", bad)
        assert wire.repeat_last_n_resolved() is None


def test_penalty_defaults_and_env(monkeypatch):
    assert wire.diag_repetition_penalty(ModelHint()) == 1.05
    assert wire.diag_repetition_penalty(ModelHint(moe=True)) == 1.03
    assert wire.diag_repetition_penalty(ModelHint(moe=True, bf16=True)) == 1.03
    monkeypatch.setenv("LUMEN_REPETITION_PENALTY", "1.2")
    assert wire.diag_repetition_penalty(ModelHint()) == pytest.approx(1.2)
    for bad in ("0", "-1", "nan", "inf", "x"):
        monkeypatch.setenv("LUMEN_REPETITION_PENALTY", bad)
        assert wire.diag_repetition_penalty(ModelHint()) == 1.05
    assert wire.frequency_penalty_resolved() == 0.0
    monkeypatch.setenv("LUMEN_FREQUENCY_PENALTY", "0.4")
    assert wire.frequency_penalty_resolved() == pytest.approx(0.4)
    monkeypatch.setenv("LUMEN_FREQUENCY_PENALTY", "-0.4")
    assert wire.frequency_penalty_resolved() == 0.0


def test_anti_restate_default(monkeypatch):
    # runtime_defaults.rs:970-999: on only for a BF16 MoE unless overridden
    assert wire.anti_restate_default(ModelHint()) is False
    assert wire.anti_restate_default(ModelHint(moe=True)) is False
    assert wire.anti_restate_default(ModelHint(moe=True, bf16=True)) is True
    monkeypatch.setenv("LUMEN_ANTI_RESTATE", "off")
    assert wire.anti_restate_default(ModelHint(moe=True, bf16=True)) is False
    monkeypatch.setenv("LUMEN_ANTI_RESTATE", "1")
    assert wire.anti_restate_default(ModelHint()) is True


def test_request_to_sampling_params(monkeypatch):
    p = wire.sampling_from_request({})
    assert p.temperature == pytest.approx(0.7)
    assert p.seed is not None and p.top_p is None and p.top_k is None
    assert p.repetition_penalty == 1.05 and p.presence_penalty is None
    assert p.frequency_penalty == 0.0 and p.repeat_last_n is None and p.anti_restate is False
    q = wire.sampling_from_request({"temperature": 0, "seed": 7, "top_p": 0.9, "top_k": 40,
                                    "min_p": 0.05, "presence_penalty": 0.0,
                                    "frequency_penalty": 0.3})
    assert q.temperature == 0.0 and q.seed == 7 and q.top_k == 40
    assert q.top_p == pytest.approx(0.9) and q.min_p == pytest.approx(0.05)
    assert q.presence_penalty is None and q.frequency_penalty == pytest.approx(0.3)
    # two requests without a seed get different seeds
    assert wire.sampling_from_request({}).seed != wire.sampling_from_request({}).seed
    for bad, field in (({"temperature": 2.5}, "temperature"), ({"temperature": float("nan")},
                       "temperature"), ({"top_p": 1.5}, "top_p"), ({"top_p": -0.1}, "top_p")):
        with pytest.raises(wire.WireError) as e:
            wire.sampling_from_request(bad)
        assert e.value.field == field
