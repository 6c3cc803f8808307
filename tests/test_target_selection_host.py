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
