"""CPU checks of the graph-bias oracle (oracle/bias_ref.py) and of the host
part of bozo_amd/bias.py (edge collapsing by content)."""
import numpy as np

from oracle import bias_ref as R


def dense_local(edge_map, alpha, contents, W):
    """Independent formulation: a dense weight matrix over the distinct
    contents, gathered by (key, query) index pairs."""
    u = sorted(set(contents))
    ix = {c: i for i, c in enumerate(u)}
    M = np.zeros((len(u), len(u)))
    for (s, d), wgt in edge_map.items():
        if s in ix and d in ix:
            M[ix[s], ix[d]] = wgt
    T = len(contents)
    c = np.array([ix[x] for x in contents])
    t = np.arange(T)[:, None]
    s = t - (W - np.arange(W)[None, :])
    ok = s >= 0
    wgt = np.where(ok, M[c[np.clip(s, 0, None)], c[t]], 0.0)
    return np.where(wgt > 0, alpha * wgt, 0.0)


def test_local_bias_oracle_vs_dense():
    r = np.random.default_rng(0)
    contents = [f"c{i}" for i in r.integers(0, 9, 40)]
    edge_map = {(f"c{a}", f"c{b}"): float(r.random() - 0.2) for a in range(9) for b in range(9)
                if r.random() < 0.5}
    bias, (hits, mx, mean) = R.local_bias(edge_map, 0.7, contents, 6, batch=2, dtype=np.float64)
    ref = dense_local(edge_map, 0.7, contents, 6)
    assert np.allclose(bias[0], ref) and np.allclose(bias[1], ref)
    pos = ref[ref > 0] / 0.7
    assert hits == pos.size and abs(mx - pos.max()) < 1e-12 and abs(mean - pos.mean()) < 1e-12


def test_global_bias_oracle_is_strictly_causal():
    contents = ["a", "b", "a", "c", "b"]
    edge_map = {("a", "b"): 0.5, ("b", "a"): 0.25, ("a", "a"): 0.1, ("c", "b"): -1.0}
    bias, (hits, mx, mean) = R.global_bias(edge_map, 2.0, contents, dtype=np.float64)
    b = bias[0]
    assert np.all(np.triu(b) == 0)
    assert b[1, 0] == 1.0 and b[2, 1] == 0.5 and b[2, 0] == 0.2 and b[4, 2] == 1.0 and b[4, 3] == 0.0
    assert hits == 5 and mx == 0.5


class _E:
    def __init__(self, src, dst, weight, relation="tension"):
        self.src, self.dst, self.weight, self.relation = src, dst, weight, relation


class _G:
    def __init__(self, edges):
        self.edges = edges


def test_from_graph_collapses_by_content_with_max():
    from bozo_amd.bias import GraphBias
    g = _G([_E("a#1", "b#2", 0.3), _E("a#7", "b#9", 0.6), _E("a#3", "b#4", 0.5),
            _E("a#1", "b#2", 0.9, relation="other"), _E("x", "y#1", 0.2), _E("p#1", "q", -0.5)])
    gb = GraphBias.from_graph(g, alpha=0.5)
    assert gb.edge_map == {("a", "b"): 0.6, ("x", "y"): 0.2}
    assert gb.lookup("a", "b") == 0.6 and gb.lookup("b", "a") == 0.0
