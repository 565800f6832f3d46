"""hearth_amd.generate on the real library (libhearth.so on the GPU).

- greedy speculative generation equals plain greedy generation token for token (the
  reference checks the same on its own library, tests/py/test_runtime.py:3412-3419),
  with and without the repetition penalty, on the tiny Qwen3-MoE model and the
  DeepSeek-V3-routed variant;
- a sampled speculative generation is reproducible for a fixed seed and leaves the KV
  of the sequence it yielded (the next logits equal a fresh evaluation's bits);
- Sampler.probs / argmax / sample on the device equal the CPU restatement on the same
  logits.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle_py as O
from hearth_amd import container
from hearth_amd.engine import Engine
from hearth_amd.generate import Sampler, generate, generate_ids

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _prompt(vocab):
    base = [int(t) for t in container.uniform_ints(31, 12, vocab)]
    return base * 3 + base[:5]


@pytest.mark.parametrize("which", ["tiny", "dsv3"])
def test_greedy_speculative_equals_plain_on_gpu(which, tiny_model, variant_models):
    path = tiny_model if which == "tiny" else variant_models("dsv3")
    with Engine(path, max_seq=512) as e:
        prompt = _prompt(e.vocab_size)
        for s in (Sampler.greedy(), Sampler(temperature=0.0, repetition_penalty=1.3)):
            plain, s1 = generate_ids(e, prompt, 48, s)
            drafted = 0
            for draft_len, n in ((4, 3), (8, 2), (1, 1)):
                spec, s2 = generate_ids(e, prompt, 48, s, (), "ngram", draft_len, n)
                assert spec == plain, (which, s, draft_len, n)
                assert s2.finish_reason == s1.finish_reason == "length"
                assert s2.forwards + s2.accepted == s1.forwards
                assert e.pos == len(prompt) + len(spec) - 1
                drafted += s2.drafted
            assert drafted > 0


def test_sampled_speculative_generation_on_gpu(tiny_model):
    with Engine(tiny_model, max_seq=512) as e:
        prompt = _prompt(e.vocab_size)
        drafted = 0
        # narrow settings, so that the sampled text falls into loops the n-gram lookup drafts from
        for kw in (dict(temperature=0.6, top_k=2), dict(temperature=0.9, top_k=3, min_p=0.5, repetition_penalty=1.02)):
            a, sa = generate_ids(e, prompt, 40, Sampler(seed=5, **kw), (), "ngram", 6, 3)
            nxt = e.eval([a[-1]])
            seq = prompt + a
            e.reset()
            e.eval(seq[:-1])
            assert np.array_equal(_bits(nxt), _bits(e.eval([seq[-1]])))
            b, sb = generate_ids(e, prompt, 40, Sampler(seed=5, **kw), (), "ngram", 6, 3)
            assert a == b and (sa.drafted, sa.accepted) == (sb.drafted, sb.accepted)
            drafted += sa.drafted
            # prefix reuse: the same sample from a warm engine holding the prompt
            gen = generate(e, prompt, 40, Sampler(seed=5, **kw), (), "ngram", 6, 3, held=seq[:e.pos])
            assert [t.id for t in gen] == a
        assert drafted > 0


def test_sampler_methods_on_gpu():
    rng = np.random.default_rng(8)
    for V in (7, 300, 4096):
        x = rng.normal(0, 2, V).astype(np.float32)
        ctx = rng.integers(0, V, 9)
        for kw in (dict(temperature=0.8, top_p=0.9), dict(temperature=1.2, top_k=5, min_p=0.05),
                   dict(temperature=0.0, repetition_penalty=1.5), dict(temperature=0.7, repetition_penalty=1.4)):
            s = Sampler(seed=3, **kw)
            c = ctx if s.uses_context else ()
            rc, want = O.probs_s(x, O.sampler(context=c, **{k: v for k, v in kw.items()}))
            assert rc == 0
            assert np.array_equal(s.probs(x, ctx), want)
            rc, g = O.probs_s(x, O.sampler(0.0, repetition_penalty=s.repetition_penalty, context=c))
            assert s.argmax(x, ctx) == int(np.argmax(g))
            u = np.random.default_rng(3).random()
            tok = s.sample(x, ctx)
            if s.is_greedy:
                assert tok == int(np.argmax(g))
            else:
                assert tok == O.lib().ho_draw(np.ascontiguousarray(want).ctypes.data_as(O._DP), V, u)
    with pytest.raises(ValueError):
        Sampler().probs(np.array([np.nan, 1.0], dtype=np.float32))


def test_cli_run_and_bench_on_gpu(tiny_model, tmp_path, capsys):
    import json
    from hearth_amd.cli import main
    ids = ",".join(str(t) for t in _prompt(container.TINY.vocab))
    outs = []
    for spec in ("none", "ngram"):
        out = tmp_path / f"run_{spec}.json"
        assert main(["run", str(tiny_model), "--ids", ids, "-n", "24", "--ignore-eos", "--speculative", spec,
                     "--json-out", str(out), "--max-seq", "256"]) == 0
        outs.append(json.loads(out.read_text()))
    assert outs[0]["output_ids"] == outs[1]["output_ids"] and len(outs[0]["output_ids"]) == 24
    assert outs[1]["stats"]["drafted"] > 0 and outs[0]["stats"]["drafted"] == 0
    capsys.readouterr()
    assert main(["bench", str(tiny_model), "--prompt-tokens", "32", "--gen-tokens", "24", "--ids", "greedy",
                 "--speculative", "ngram", "--draft-len", "6", "--json", "--max-seq", "256"]) == 0
    res = json.loads(capsys.readouterr().out)
    for key in ("model", "arch", "params_total", "params_active", "isa", "threads", "io_threads", "cache_slots",
                "options", "ids", "route_replay", "prefill_tokens", "prefill_s", "prefill_tok_s", "decode_tokens",
                "decode_s", "decode_tok_s", "prefill_stats", "decode_stats", "verify"):
        assert key in res, key
    v = res["verify"]
    assert v["forwards"] >= 1 and 0 <= v["accepted"] <= v["drafted"] and v["tokens_per_forward"] >= 1.0
