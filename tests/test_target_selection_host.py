"""Route selection of the Target drop-in on the host, against the oracle.

The oracle's ``select_best`` and ``sample_route`` are pinned by the
reference's literals and the closed form of the seeded draw
(``tests/test_oracle_pinning.py``); here the drop-in's own ``_select_route``
(policies ``target_best`` and ``target_sample``) must pick the same route as
the oracle on seeded random score lists: ties in the selection score, in the
draft path log-prob and in the route id order, routes sharing token paths,
``-inf`` and ``+inf`` scores, several temperatures, seeds and rounds.  The
draw's reported uniform must be the oracle's, and the inputs' order must not
matter."""

import math
import random

import pytest

from helpers import pkg
from oracle import scoring as osc


def _backend(policy, temperature=1.0):
    tr = pkg("target_runtime")
    b = object.__new__(tr.DirectFlashInferMaskedTreeVerifyBackend)
    b.route_selection_policy = policy
    b.route_sampling_temperature = temperature
    b.score_weights = None
    return b


def _random_scores(rng):
    ty = pkg("types")
    n = rng.randint(1, 9)
    pool = [-0.5, -1.0, -1.25, -2.0, -math.inf]
    scores = []
    for i in range(n):
        path = tuple(rng.randint(0, 3) for _ in range(rng.randint(1, 4)))
        sel = rng.choice(pool + [rng.uniform(-6.0, 0.0)])
        draft = rng.choice([-0.25, -0.5, rng.uniform(-3.0, 0.0)])
        rid = rng.randint(0, 40)
        while any(s.route_id == rid for s in scores):
            rid = rng.randint(0, 40)
        scores.append(ty.TargetRouteScore(route_id=rid, token_ids=path, target_logprob=sel, draft_logprob=draft,
                                          token_logprobs=(sel,), first_token_logprob=sel, selection_score=sel))
    if rng.random() < 0.1:
        k = rng.randrange(n)
        s = scores[k]
        scores[k] = ty.TargetRouteScore(route_id=s.route_id, token_ids=s.token_ids, target_logprob=math.inf,
                                        draft_logprob=s.draft_logprob, selection_score=math.inf)
    return scores


def _as_dicts(scores):
    return [dict(route_id=s.route_id, token_ids=s.token_ids, selection_score=float(s.selection_score),
                 draft_path_logprob=s.draft_path_logprob) for s in scores]


def test_target_best_matches_oracle():
    b = _backend("target_best")
    for seed in range(300):
        rng = random.Random(seed)
        scores = _random_scores(rng)
        got = b._select_route(scores)
        assert got.route_id == osc.select_best(_as_dicts(scores))["route_id"], f"seed {seed}"


def test_target_sample_matches_oracle():
    picked = set()
    for seed in range(300):
        rng = random.Random(1000 + seed)
        scores = _random_scores(rng)
        temperature = rng.choice([1.0, 0.5, 2.0])
        draw_seed, draw_round = rng.randint(0, 1 << 40), rng.randint(0, 1000)
        b = _backend("target_sample", temperature)
        got, meta = b._select_route_with_metadata(scores, route_sampling_seed=draw_seed,
                                                  route_sampling_round=draw_round)
        want, draw = osc.sample_route(_as_dicts(scores), draw_seed, draw_round, temperature)
        assert got.route_id == want["route_id"] and meta["route_sampling_uniform"] == draw, f"seed {seed}"
        shuffled = list(scores)
        rng.shuffle(shuffled)
        again = b._select_route(shuffled, route_sampling_seed=draw_seed, route_sampling_round=draw_round)
        assert again.route_id == got.route_id, f"seed {seed}: input order changed the draw"
        picked.add(sorted(_as_dicts(scores), key=lambda s: (s["token_ids"], s["draft_path_logprob"],
                                                            s["selection_score"], s["route_id"])).index(
            next(d for d in _as_dicts(scores) if d["route_id"] == got.route_id)))
    assert len(picked) > 3  # the draws land on many positions of the canonical order


def test_target_sample_refusals():
    ty = pkg("types")
    s = [ty.TargetRouteScore(route_id=1, token_ids=(1,), target_logprob=-1.0, draft_logprob=0.0, selection_score=-1.0)]
    b = _backend("target_sample")
    with pytest.raises(ValueError):
        b._select_route(s)  # seed and round are required
    with pytest.raises(ValueError):
        b._select_route(s, route_sampling_seed=1, route_sampling_round=-1)
    nan = [ty.TargetRouteScore(route_id=1, token_ids=(1,), target_logprob=math.nan, draft_logprob=0.0,
                               selection_score=math.nan)]
    with pytest.raises(ValueError):
        b._select_route(nan, route_sampling_seed=1, route_sampling_round=0)


def test_truncation_matches_oracle_and_reference_literal():
    """``_truncate_selected_path`` (target_runtime.py:675-700): the reference
    literal (tests/test_target_kv_commit.py:345-367), then seeded random paths,
    limits and EOS ids against the oracle, refusals included."""
    tr = pkg("target_runtime")
    cut = tr.DirectFlashInferMaskedTreeVerifyBackend._truncate_selected_path
    assert cut(token_ids=(10, 11, 12, 13), node_ids=(20, 21, 22, 23), max_tokens=3, eos_token_id=11) == \
        ((10, 11), (20, 21))
    rng = random.Random(5)
    for _ in range(500):
        n = rng.randint(1, 6)
        toks = tuple(rng.randint(0, 5) for _ in range(n))
        nodes = tuple(range(100, 100 + n))
        limit = rng.choice([None, 1, 2, 3, 8])
        eos = rng.choice([None, 0, 3, 9])
        assert cut(token_ids=toks, node_ids=nodes, max_tokens=limit, eos_token_id=eos) == \
            osc.truncate_path(toks, nodes, limit, eos)
    for bad in (dict(token_ids=(), node_ids=(), max_tokens=None, eos_token_id=None),
                dict(token_ids=(1, 2), node_ids=(3,), max_tokens=None, eos_token_id=None),
                dict(token_ids=(1,), node_ids=(3,), max_tokens=0, eos_token_id=None)):
        with pytest.raises(ValueError):
            cut(**bad)


def test_weights_and_fallback_reasons():
    """Score weights must match the route depth; a selected route below the
    first-token or the path threshold gives the reference's fallback reason
    (target_runtime.py:708-720 order: first token first)."""
    ty = pkg("types")
    b = _backend("target_best")
    b.score_weights = (0.5, 0.25)
    assert b._weights_for_depth(2) == (0.5, 0.25)
    with pytest.raises(ValueError):
        b._weights_for_depth(3)
    s = ty.TargetRouteScore(route_id=1, token_ids=(1, 2), target_logprob=-3.0, draft_logprob=0.0,
                            first_token_logprob=-2.0, selection_score=-3.0)
    b.first_token_threshold, b.fallback_threshold = None, None
    assert b._fallback_reason(s) is None
    b.fallback_threshold = -2.5
    assert b._fallback_reason(s) == "path_score_below_threshold"
    b.first_token_threshold = -1.0
    assert b._fallback_reason(s) == "first_token_below_threshold"
    b.first_token_threshold, b.fallback_threshold = -2.0, -3.0
    assert b._fallback_reason(s) is None  # equal to a threshold is not below it


def test_route_score_fast_constructor_equals_dataclass():
    """The scoring loop's constructor gives the same frozen object as the
    dataclass's own __init__ for a keyword set naming every field."""
    import dataclasses

    tr = pkg("target_runtime")
    ty = pkg("types")
    fields = dict(route_id=3, token_ids=(5, 6), target_logprob=-1.5, draft_logprob=-0.25, token_logprobs=(-1.0, -0.5),
                  first_token_logprob=-1.0, selection_score=-1.5, score_weights=(), draft_token_logprobs=(-0.1, -0.15))
    assert set(fields) == {f.name for f in dataclasses.fields(ty.TargetRouteScore)}
    fast, slow = tr._route_score(**fields), ty.TargetRouteScore(**fields)
    assert fast == slow and hash(fast) == hash(slow) and repr(fast) == repr(slow)
    assert fast.draft_path_logprob == slow.draft_path_logprob
    with pytest.raises(dataclasses.FrozenInstanceError):
        fast.route_id = 4
