"""Route selection on the device (atlas_route_select) against the host
selection of the Target runtime, which follows the reference's
verify_payloads (src/atlas_0709/target_runtime.py:567-573, :722-765,
:754-760), and against the oracle's select_best: the same selected route,
committed count and commit positions on seeded cases with ties, NaN and
infinite log-probs, weights, thresholds, truncated routes, both policies and
the three roundings."""

import math
import random

import numpy as np
import pytest
import torch

from helpers import pkg

pytestmark = pytest.mark.gpu


def _oracle_index(routes, values, dtype, d, policy, weights):
    """Index of the route the oracle selects: per-token values rounded to
    the logits dtype, the score a left-to-right float sum (or the weighted
    sum), then oracle.scoring.select_best (target_best) or route 0."""
    from oracle import scoring as osc

    if policy == "first_route":
        return 0
    if dtype == torch.float16:
        vals = values.astype(np.float16).astype(np.float32).tolist()
    elif dtype == torch.bfloat16:
        vals = torch.from_numpy(values.copy()).to(torch.bfloat16).float().tolist()
    else:
        vals = values.tolist()
    k = len(routes)
    dicts = []
    for i, r in enumerate(routes):
        lps = [vals[i]] + vals[k + i * (d - 1): k + (i + 1) * (d - 1)]
        sel = sum(lps) if weights is None else sum(w * v for w, v in zip(weights, lps))
        draft = float(sum(r.draft_token_logprobs)) if r.draft_token_logprobs else float(r.draft_logprob)
        dicts.append(dict(index=i, route_id=r.route_id, selection_score=sel, draft_path_logprob=draft))
    return osc.select_best(dicts)["index"]


def _rounded(values, dtype):
    """The fp32 values rounded to the logits dtype (what the host reads)."""
    if dtype == torch.float16:
        return values.astype(np.float16).astype(np.float32)
    if dtype == torch.bfloat16:
        return torch.from_numpy(values.copy()).to(torch.bfloat16).float().numpy()
    return values.copy()


def _score_key(score):
    """A TargetRouteScore's fields with NaN made comparable."""
    def fix(v):
        if isinstance(v, float) and math.isnan(v):
            return "nan"
        if isinstance(v, tuple):
            return tuple(fix(x) for x in v)
        return v
    return tuple(sorted((k, fix(v)) for k, v in vars(score).items()))


def _backend(policy, weights, thr_path, thr_first):
    tr = pkg("target_runtime")
    b = object.__new__(tr.DirectFlashInferMaskedTreeVerifyBackend)
    b.route_selection_policy = policy
    b.score_weights = weights
    b.fallback_threshold = thr_path
    b.first_token_threshold = thr_first
    b.match_logits_dtype_rounding = True
    b.route_sampling_temperature = 1.0
    return b


def _value(rng, pool):
    r = rng.random()
    if r < 0.04:
        return math.nan
    if r < 0.07:
        return -math.inf
    if r < 0.4:
        return rng.choice(pool)  # repeated values: ties after summing
    return -rng.random() * 12.0


def _case(rng, k, d):
    tr = pkg("target_runtime")
    pool = [-0.5, -1.25, -3.0, -0.0, -7.5]
    ids = rng.sample(range(-50, 1000), k)
    routes = []
    for r in range(k):
        if rng.random() < 0.5:
            drafts = tuple(rng.choice([-0.25, -1.0, -2.0, 0.0]) for _ in range(d))
            routes.append(tr.VerifyRoutePayload(route_id=ids[r], token_ids=tuple(range(d)), draft_logprob=-9.0,
                                                draft_token_logprobs=drafts))
        else:
            routes.append(tr.VerifyRoutePayload(route_id=ids[r], token_ids=tuple(range(d)),
                                                draft_logprob=rng.choice([-1.0, -2.5, 0.0])))
    n = k + k * (d - 1)
    values = np.asarray([_value(rng, pool) for _ in range(n)], dtype=np.float32)
    return routes, values


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_device_selection_matches_host_selection(dev, dtype):
    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    rng = random.Random({torch.float16: 1, torch.bfloat16: 2, torch.float32: 3}[dtype])
    mapped = lib_mod.MappedReadback(lib_mod.SELECT_MAX_ENTRIES + 2)
    mapped.np[:] = np.nan
    checked = fallbacks = 0
    for case in range(400):
        k, d = rng.randint(1, 12), rng.randint(1, 6)
        policy = "first_route" if case % 7 == 0 else "target_best"
        weights = None
        if policy == "target_best" and case % 3 == 0:
            weights = tuple(rng.choice([1.0, 0.5, 0.25, 2.0, 0.1]) for _ in range(d))
        thr_path = thr_first = None
        if policy == "target_best" and case % 4 == 1:
            thr_path = rng.choice([-6.0, -15.0, -1.0])
        if policy == "target_best" and case % 5 == 2:
            thr_first = rng.choice([-3.0, -8.0])
        b = _backend(policy, weights, thr_path, thr_first)
        routes, values = _case(rng, k, d)
        paths = [r.token_ids for r in routes]
        nodes = [[rng.randrange(0, 40) for _ in range(d)] for _ in range(k)]
        commit_lens = [rng.randint(1, d) for _ in range(k)]
        prefix = rng.randrange(0, 5000)
        inputs = b._device_selection_inputs(routes, paths, nodes)
        assert inputs is not None
        # host: the runtime's scores and selection from the same values
        scores = b._route_scores_from_values(routes, paths, values.copy(), dtype)
        selected, _ = b._select_route_with_metadata(scores)
        host_idx = next(i for i, r in enumerate(routes) if r.route_id == selected.route_id)
        reason = b._fallback_reason(selected)
        host_count = 0 if reason is not None else commit_lens[host_idx]
        # the oracle's selection (oracle/scoring.py) from the values read in the logits dtype
        assert host_idx == _oracle_index(routes, values, dtype, d, policy, weights)
        # device
        buf = torch.empty(len(values) + 2, dtype=torch.float32, device=dev)
        buf[: len(values)] = torch.from_numpy(values).to(dev)
        pos = torch.full((2 * d,), -1, dtype=torch.int64, device=dev)
        policy_code, w, draft, route_ids, flat_nodes = inputs
        import ctypes

        rc = lib.atlas_route_select(
            lib_mod.ptr(buf), k, d, policy_code, b._rounding_code(dtype),
            (ctypes.c_double * d)(*w) if w is not None else None, 0 if w is None else d,
            (ctypes.c_double * k)(*draft), (ctypes.c_int64 * k)(*route_ids), (ctypes.c_int32 * k)(*commit_lens),
            (ctypes.c_int32 * (k * d))(*flat_nodes), int(thr_path is not None), float(thr_path or 0.0),
            int(thr_first is not None), float(thr_first or 0.0), prefix, lib_mod.ptr(pos), lib_mod.ptr(pos[d:]),
            lib_mod.ptr(buf[len(values):]), mapped.device_ptr if case % 2 else None, lib_mod.stream_of(dev))
        lib_mod.check(rc, "atlas_route_select")
        torch.cuda.synchronize()
        dev_idx, dev_count = buf[len(values):].view(torch.int32).tolist()
        assert (dev_idx, dev_count) == (host_idx, host_count), (case, k, d, policy, weights, thr_path, thr_first)
        if case % 2:
            # the values rounded to the logits dtype, as the host rounds them, and the result,
            # written by the launch to mapped host memory
            nv = len(values)
            got = mapped.np[:nv].copy()
            exp = _rounded(values, dtype)
            nan = np.isnan(exp)
            assert (np.isnan(got) == nan).all()
            assert (got[~nan].view(np.uint32) == exp[~nan].view(np.uint32)).all()
            assert mapped.np[nv:nv + 2].view(np.int32).tolist() == [host_idx, host_count]
            # and the scores built from them without rounding again equal the host's
            again = b._route_scores_from_values(routes, paths, got, dtype, rounded=True)
            assert [_score_key(x) for x in again] == [_score_key(x) for x in scores]
            mapped.np[:] = np.nan
        src, dst = pos[:d].tolist(), pos[d:].tolist()
        assert dst == [prefix + i for i in range(d)]
        assert src == [prefix + nodes[host_idx][i] if i < host_count else prefix + i for i in range(d)]
        checked += 1
        fallbacks += host_count == 0
    assert checked == 400 and 0 < fallbacks < 400


def test_device_selection_refusals(dev):
    """Sizes beyond the launch's limits and bad codes are refused before any
    launch (the runtime then selects on the host)."""
    import ctypes

    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    buf = torch.zeros(64, dtype=torch.float32, device=dev)
    pos = torch.zeros(64, dtype=torch.int64, device=dev)

    def call(k, d, policy=0, rounding=0, lens=None, nodes=None):
        lens = lens or [1] * k
        nodes = nodes or [0] * (k * d)
        return lib.atlas_route_select(
            lib_mod.ptr(buf), k, d, policy, rounding, None, 0, (ctypes.c_double * max(k, 1))(),
            (ctypes.c_int64 * max(k, 1))(), (ctypes.c_int32 * max(k, 1))(*lens), (ctypes.c_int32 * max(k * d, 1))(*nodes),
            0, 0.0, 0, 0.0, 0, lib_mod.ptr(pos), lib_mod.ptr(pos[32:]), lib_mod.ptr(buf[60:]), None,
            lib_mod.stream_of(dev))

    einval = lib_mod.ATLAS_EINVAL
    assert call(65, 1) == einval and call(0, 1) == einval and call(4, 17) == einval
    assert call(40, 13) == einval  # 520 entries
    assert call(2, 2, policy=2) == einval and call(2, 2, rounding=3) == einval
    assert call(2, 2, lens=[3, 1]) == einval and call(2, 2, nodes=[0, 1, 40000, 2]) == einval
    assert call(2, 2) == lib_mod.ATLAS_OK
    torch.cuda.synchronize()
