"""The continuous-batching engine (rkv_engine_*) on the GPU: every request's
tokens equal what the CPU oracle decoder generates for that request alone,
however the scheduler batches, pauses and resumes it.

The engine runs a request's prompt through causal prefill attention in one
step and then decodes inside mixed batches; the oracle feeds the prompt one
token at a time.  Both are within the fp32 attention tolerance of each other,
so the greedy tokens agree unless two logits tie within ~1e-5 (the test
prints the smallest top-1 / top-2 margin it relies on).
"""
import numpy as np
import pytest

import oracle
from rustral_amd import model
from rustral_amd._lib import RKV_ERR_OOM, RkvError
from rustral_amd.serving import LOW, NORMAL
from tests.gpu_util import say

pytestmark = pytest.mark.gpu

EOS = 2


def expected(params, prompt, max_tokens):
    """Oracle tokens for one request, cut after the first EOS as the
    scheduler completes a request (Request::should_complete)."""
    toks, lg = oracle.decoder_generate(oracle.decoder_config(), params, prompt, max_tokens,
                                       logits=True)
    toks = toks.tolist()
    if EOS in toks:
        toks = toks[:toks.index(EOS) + 1]
    srt = np.sort(lg[:len(toks)], axis=1)
    return toks, float((srt[:, -1] - srt[:, -2]).min())


def requests(seed, lens, max_tokens):
    rng = np.random.default_rng(seed)
    return [(rng.integers(0, 1000, n).astype(np.int32), m) for n, m in zip(lens, max_tokens)]


def test_engine_requests_match_oracle(dev):
    say("engine: 8 requests, max batch 4")
    cfg = model.config()
    params = model.init_params(cfg, seed=0, std=0.02)
    reqs = requests(1, [5, 20, 33, 1, 12, 40, 7, 64], [10, 25, 8, 30, 16, 12, 20, 9])
    eng = model.Engine(cfg, params, num_blocks=64, max_batch_size=4)
    ids = [eng.submit(p, m) for p, m in reqs]
    steps = eng.run()
    assert steps > 0
    st = eng.scheduler.stats()
    assert st["completed"] == len(reqs) and st["running"] == 0 and st["pending"] == 0
    margins = []
    for rid, (p, m) in zip(ids, reqs):
        want, margin = expected(params, p, m)
        margins.append(margin)
        assert eng.generated(rid) == want, f"request {rid}"
    say(f"smallest top-1/top-2 logit margin {min(margins):.3e}")


def test_engine_preempted_requests_recompute_to_the_same_tokens(dev):
    """Low-priority requests are paused under batch pressure and resumed by
    recomputing prompt + generated tokens; their tokens do not change."""
    say("engine: preemption and recompute")
    cfg = model.config()
    params = model.init_params(cfg, seed=0, std=0.02)
    reqs = requests(2, [9, 30, 14, 22, 6], [20, 12, 18, 15, 24])
    prio = [NORMAL, LOW, NORMAL, LOW, NORMAL]
    eng = model.Engine(cfg, params, num_blocks=64, max_batch_size=4)
    ids = [eng.submit(p, m, pr) for (p, m), pr in zip(reqs, prio)]
    paused_seen = 0
    for _ in range(500):
        if eng.step() == 0:
            break
        paused_seen = max(paused_seen, eng.scheduler.stats()["paused"])
    assert eng.scheduler.stats()["completed"] == len(reqs)
    assert paused_seen > 0, "the scenario is meant to preempt"
    for rid, (p, m) in zip(ids, reqs):
        want, _ = expected(params, p, m)
        assert eng.generated(rid) == want, f"request {rid}"


def test_engine_reports_pool_exhaustion(dev):
    say("engine: KV pool exhaustion")
    cfg = model.config()
    params = model.init_params(cfg, seed=0, std=0.02)
    eng = model.Engine(cfg, params, num_blocks=3, max_batch_size=2)
    (p, _), = requests(3, [40], [1])
    eng.submit(p, 20)
    with pytest.raises(RkvError) as e:
        for _ in range(30):
            if eng.step() == 0:
                break
    assert e.value.code == RKV_ERR_OOM


def test_engine_steps_on_after_an_out_of_memory_update(dev):
    """An update that finds no free block raises RKV_ERR_OOM; the engine keeps
    stepping: the starved request is paused (its blocks go back), the other
    request's rows never read past a table, and the starved one resumes by
    recompute.  Every request's tokens still equal the oracle's."""
    say("engine: steps after an out-of-memory update")
    cfg = model.config()
    params = model.init_params(cfg, seed=0, std=0.02)
    reqs = requests(4, [16, 30], [30, 20])
    eng = model.Engine(cfg, params, num_blocks=5, max_batch_size=2)
    ids = [eng.submit(p, m) for p, m in reqs]
    ooms = 0
    for _ in range(200):
        try:
            if eng.step() == 0:
                break
        except RkvError as e:
            assert e.code == RKV_ERR_OOM
            ooms += 1
    assert ooms >= 1, "the scenario is meant to run out of blocks"
    assert eng.scheduler.stats()["completed"] == len(reqs)
    for rid, (p, m) in zip(ids, reqs):
        want, _ = expected(params, p, m)
        assert eng.generated(rid) == want, f"request {rid}"


def _config0_fixture():
    import os
    rows = {}
    for line in open(os.path.join(os.path.dirname(__file__), "golden", "config0_tokens.txt")):
        if not line.startswith("#"):
            key, *vals = line.split()
            rows[key] = [int(v) for v in vals]
    return np.array(rows["prompt"], np.int32), rows["tokens"]


def test_config0_fixture_through_decoder_and_engine(dev):
    """What rust/rustral-rocm-backend/tests/model_parity.rs asserts, through
    the same entry points: the decoder's tokens equal the committed oracle
    fixture, one token at a time over a growing prefix too, and the engine
    generates them for the same request beside a second one."""
    say("config0 fixture: decoder, generate_token, engine")
    cfg = model.config()
    params = model.init_params(cfg, seed=0, std=0.02)
    prompt, want = _config0_fixture()
    dec = model.Decoder(cfg, params)
    assert dec.generate(prompt, 64).tolist() == want
    assert dec.generate(prompt, 64).tolist() == want
    prefix = prompt.tolist()
    for t in want[:8]:
        assert int(dec.generate(np.array(prefix, np.int32), 1)[0]) == t
        prefix.append(t)
    eng = model.Engine(cfg, params, num_blocks=64, max_batch_size=4)
    rid = eng.submit(prompt, 64)
    other = eng.submit(prompt[:5], 10)
    assert eng.run() >= 64
    st = eng.scheduler.stats()
    assert st["pending"] == st["running"] == st["paused"] == 0
    assert eng.generated(rid) == want
    assert len(eng.generated(other)) == 10
    assert (st["completed"], st["total_tokens_generated"]) == (2, 74)
