"""CPU checks of the tau-export oracle (oracle/export_ref.py) and the graph
container (bozo_amd/export.py).  The oracle's numpy reductions are pinned by
loops written from the definitions: the order-statistic definition of the
linear quantile, first arg-max, the pairwise-difference form of the Gini
coefficient, and the masked head mean."""
import itertools
import json
import math

import numpy as np
import pytest

from oracle import export_ref as X


def rnd_tau(seed, B, T, H, W, peaky=False):
    r = np.random.default_rng(seed)
    t = r.random((B, T, H, W)).astype(np.float32)
    if peaky:
        t = t ** 6
    t[:, :, :, 1] = t[:, :, :, 2]  # ties for the arg-max
    return t


def loops_stats(tau, valid_only):
    B, T, H, W = tau.shape
    out = np.zeros((H, 4))
    for h in range(H):
        vals = []
        rmax, rarg = 0.0, 0.0
        for t in range(T):
            row = []
            for w in range(W):
                v = float(np.float32(tau[:, t, h, w].mean()))
                if valid_only and t + w < W:
                    v = 0.0
                row.append(v)
            m = max(row)
            rmax += m
            rarg += row.index(m)  # first occurrence
            vals.extend(row)
        s = sorted(vals)
        n = len(s)
        g = 0.99 * (n - 1)
        k = int(math.floor(g))
        hi = s[min(k + 1, n - 1)]
        out[h] = [sum(vals) / n, s[k] + (g - k) * (hi - s[k]), rarg / T, rmax / T]
    return out


@pytest.mark.parametrize("valid_only", [False, True])
@pytest.mark.parametrize("B", [1, 3])
def test_head_stats_vs_loops(valid_only, B):
    tau = rnd_tau(1 + B, B, 13, 3, 6, peaky=True)
    got = X.head_stats([tau], valid_only)[0]
    ref = loops_stats(tau, valid_only)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6)


def test_quantile99_f32_rank_and_lerp():
    """The restated quantile keeps q, the rank and the interpolation in
    float32 (numpy >= 2 on float32 data): for n = 2056 the rank is
    float32(2055 * 0.99f) = 2034.45007, not 2034.45, which moves the result
    by 0.00007 of the gap between the two order statistics."""
    v = np.concatenate([np.zeros(2034), [0.5859375, 0.62402344], np.ones(20)]).astype(np.float32)
    g32 = np.float32(2055) * np.float32(0.99)
    assert float(g32) == 2034.4500732421875
    got = X.quantile99_f32(v)
    assert got == float(np.float32(np.float32(0.5859375) + np.float32(np.float32(0.62402344 - 0.5859375) *
                                                                       np.float32(g32 - 2034))))
    f64_rank = 0.5859375 + 0.45 * (0.62402344 - 0.5859375)  # the float64-rank value (numpy 1.x)
    assert abs(got - f64_rank) > 1e-6 and abs(got - f64_rank) < 1e-4 * (0.62402344 - 0.5859375)
    # t >= 0.5 takes numpy's other form b - (b - a)(1 - t): n = 11 gives g = 9.9
    w = np.arange(11, dtype=np.float32) / np.float32(7)
    t = np.float32(np.float32(10) * np.float32(0.99)) - np.float32(9)
    assert t >= 0.5
    assert X.quantile99_f32(w) == float(np.float32(w[10] - np.float32((w[10] - w[9]) * (np.float32(1) - t))))


@pytest.mark.skipif(int(np.__version__.split(".")[0]) < 2, reason="numpy 1.x forms the rank in float64")
def test_quantile99_f32_is_numpy_quantile():
    """The restatement equals the call the reference makes, np.quantile(vals,
    0.99) on float32 values, under this numpy (>= 2): random sizes, skewed
    values, ties."""
    r = np.random.default_rng(7)
    for n in list(range(1, 200)) + [2056, 4097, 65536]:
        for rep in range(3):
            v = (r.random(n) ** int(r.integers(1, 8))).astype(np.float32)
            if rep == 2:
                v = (np.round(v * 8) / 8).astype(np.float32)
            assert X.quantile99_f32(v) == float(np.quantile(v, 0.99)), (n, rep)


def test_gini_vs_pairwise_definition():
    r = np.random.default_rng(3)
    agg = (r.random((9, 5)) ** 3).astype(np.float32)
    gini, mean = X.concentration(agg)
    vals = agg[X.valid_mask(9, 5)].astype(np.float64)
    n = vals.size
    pair = sum(abs(a - b) for a, b in itertools.product(vals, vals)) / (2 * n * n * vals.mean())
    assert abs(gini - pair) < 1e-6
    assert abs(mean - vals.mean()) < 1e-6
    assert X.valid_mask(9, 5).sum() == sum(min(t, 5) for t in range(9))
    assert X.concentration(np.zeros((4, 3), np.float32)) == (0.0, 0.0)


def test_aggregate_vs_loops():
    taus = [rnd_tau(10 + i, 2, 7, 4, 5) for i in range(3)]
    mask = np.zeros((3, 4), bool)
    mask[0, 1] = mask[2, 3] = mask[2, 0] = True
    got = X.aggregate(taus, mask)
    ref = np.zeros((7, 5))
    for t in range(7):
        for w in range(5):
            vals = [taus[l][:, t, h, w].mean() for l in range(3) for h in range(4) if mask[l, h]]
            ref[t, w] = sum(vals) / len(vals)
    assert np.allclose(got, ref, atol=1e-6)
    everything = X.aggregate(taus, np.zeros((3, 4), bool))
    assert np.allclose(everything, np.mean([t.mean(0) for t in taus], axis=(0, 2)), atol=1e-6)


def test_edges_order_and_threshold():
    agg = np.array([[0.9, 0.9], [0.2, 0.5], [0.35, 0.1]], np.float32)
    edges, pull = X.edges(agg, 0.3)
    # W = 2: key s = t - (2 - w); t = 0 has none, t = 1 only w = 1 (s = 0)
    assert edges == [(1, 0, float(np.float32(0.5))), (2, 0, float(np.float32(0.35)))]
    assert np.allclose(pull, agg.mean(-1))


def test_classify_rules():
    assert X.classify(0.1, 0.3, 5, 0.9, 10) == "inactive"
    assert X.classify(0.1, 0.9, 5, 0.2, 10) == "diffuse"
    assert X.classify(0.1, 0.9, 8, 0.9, 10) == "syntactic"
    assert X.classify(0.1, 0.9, 2, 0.9, 10) == "long_range"
    assert X.classify(0.1, 0.9, 5, 0.9, 10) == "mid_range"


def test_graph_container_semantics(tmp_path):
    from bozo_amd.export import UniversalLivingGraph
    g = UniversalLivingGraph()
    g.upsert_node("a#0", "a", activation=0.4, metadata={"x": 1})
    g.upsert_node("a#0", "a", activation=0.3, topics=["z", "b"], metadata={"y": 2})
    assert g.nodes["a#0"].activation == 0.4 and g.nodes["a#0"].topics == ["b", "z"]
    assert g.nodes["a#0"].metadata == {"x": 1, "y": 2}
    g.upsert_node("b#1", "b")
    g.add_edge("a#0", "b#1", 0.5, metadata={"distance": 1})
    g.add_edge("a#0", "b#1", 0.4)
    g.add_edge("a#0", "b#1", 0.7, relation="other")
    g.add_edge("a#0", "b#1", 0.6)
    assert [(e.relation, e.weight) for e in g.edges] == [("tension", 0.6), ("other", 0.7)]
    assert g.density() == 2.0 and abs(g.mean_edge_weight() - 0.65) < 1e-12
    p = tmp_path / "g.json"
    g.to_json(p)
    d = json.loads(p.read_text())
    assert set(d) == {"nodes", "edges"}
    assert set(d["nodes"]["a#0"]) == {"id", "content", "topics", "activation", "stability",
                                       "base_strength", "metadata"}
    assert set(d["edges"][0]) == {"src", "dst", "weight", "relation", "metadata"}
    g2 = UniversalLivingGraph.from_json(p)
    assert g2.to_dict() == g.to_dict()
    g2.add_edge("a#0", "b#1", 0.9)
    assert len(g2.edges) == 2 and g2.edges[0].weight == 0.9
