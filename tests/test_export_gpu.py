"""Tau export reductions on the GPU (bozo_amd/export.py) against the numpy
restatement of the reference exporter (oracle/export_ref.py)."""
import numpy as np
import pytest
import torch

from bozo_amd import export as E
from oracle import export_ref as X

pytestmark = pytest.mark.gpu


class Tok:
    def id_to_token(self, i):
        return None if i % 7 == 3 else f"t{i}"


def rand_taus(seed, L, B, T, H, W, dtype):
    g = torch.Generator().manual_seed(seed)
    taus = [torch.rand(B, T, H, W, generator=g) ** (1 + 4 * l) for l in range(L)]
    return [t.to(dtype) for t in taus]


@pytest.mark.parametrize("dtype,B,valid_only", [
    (torch.float32, 1, False), (torch.bfloat16, 1, False), (torch.bfloat16, 2, True),
    (torch.float32, 3, True)])
def test_head_stats_vs_oracle(dev, dtype, B, valid_only):
    taus = rand_taus(1, 3, B, 257, 5, 64, dtype)
    got = E.head_stats([t.to(dev) for t in taus], valid_only).cpu().numpy()
    ref = X.head_stats([t.float().numpy() for t in taus], valid_only)
    assert np.allclose(got[..., [0, 2, 3]], ref[..., [0, 2, 3]], rtol=1e-5, atol=1e-6)
    assert np.max(np.abs(got[..., 1] - ref[..., 1])) <= 1e-7


def test_head_stats_many_ties_and_tiny(dev):
    # bf16 values in [0, 1] take few distinct values: long runs of equal keys
    t = (torch.rand(1, 40, 2, 8) * 4).floor().div(4).to(torch.bfloat16)
    got = E.head_stats([t.to(dev)]).cpu().numpy()
    ref = X.head_stats([t.float().numpy()])
    assert np.allclose(got, ref, atol=1e-6)
    one = torch.full((1, 1, 1, 1), 0.25)
    assert np.allclose(E.head_stats([one.to(dev)]).cpu().numpy()[0, 0], [0.25, 0.25, 0.0, 0.25])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_aggregate_vs_oracle(dev, dtype):
    taus = rand_taus(2, 4, 2, 130, 6, 16, dtype)
    mask = torch.rand(4, 6, generator=torch.Generator().manual_seed(3)) > 0.6
    got = E.aggregate_tau([t.to(dev) for t in taus], mask).cpu().numpy()
    ref = X.aggregate([t.float().numpy() for t in taus], mask.numpy())
    assert np.allclose(got, ref, atol=1e-6)
    got_all = E.aggregate_tau([t.to(dev) for t in taus], torch.zeros(4, 6, dtype=torch.bool)).cpu().numpy()
    assert np.allclose(got_all, X.aggregate([t.float().numpy() for t in taus], np.zeros((4, 6), bool)),
                       atol=1e-6)
    gini, mean = E.concentration(torch.from_numpy(ref).to(dev))
    rg, rm = X.concentration(ref)
    assert abs(gini - rg) < 1e-5 and abs(mean - rm) < 1e-6


def reference_ingest(graph, token_ids, taus, tok, thr, heads):
    """The reference ingest (export.py:162-302) over numpy arrays, built from
    the oracle's reductions."""
    T = len(token_ids)
    L, H = len(taus), taus[0].shape[2]
    W = taus[0].shape[3]
    mask = np.zeros((L, H), bool)
    for (l, h) in heads:
        mask[l, h] = True
    if not heads:
        mask[:] = True
    agg = X.aggregate([t[:, :T] for t in taus], mask)
    gini, agg_mean = X.concentration(agg)
    edges, pull = X.edges(agg, thr)
    name = lambda i: tok.id_to_token(i) or f"<{i}>"  # noqa: E731
    ei = 0
    for t in range(T):
        qid = f"{name(token_ids[t])}#{t}"
        graph.upsert_node(id=qid, content=name(token_ids[t]), activation=min(1.0, 0.3 + float(pull[t])),
                          metadata={"absolute_pos": t, "token_id": int(token_ids[t])})
        while ei < len(edges) and edges[ei][0] == t:
            _, s, wt = edges[ei]
            kid = f"{name(token_ids[s])}#{s}"
            graph.upsert_node(id=kid, content=name(token_ids[s]), activation=min(1.0, 0.3 + wt),
                              metadata={"absolute_pos": s, "token_id": int(token_ids[s])})
            graph.add_edge(src=kid, dst=qid, weight=wt, relation="tension", metadata={"distance": t - s})
            ei += 1
    return gini, agg_mean, len(edges)


def test_ingest_matches_reference_pipeline(dev):
    from bozo_amd import model as M
    cfg = M.TensionConfig(vocab_size=60, dim=64, num_layers=5, num_heads=4, window=8, max_seq_len=64,
                          dropout=0.0, global_every=5, use_rope=True)
    torch.manual_seed(0)
    m = M.TensionLM(cfg).to(dev).eval()
    with torch.no_grad():
        m.blocks[0].tension.wq.weight.mul_(20.0)  # spread the taus
    ids = torch.randint(0, 60, (1, 50), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        _, _, taus = m(ids.to(dev), return_all=True)
    # the global layer's down-sampled tau [B,T,H,min(W,T)] has the local
    # shape, so the reference's most-common-shape rule keeps all five
    local = E.TauExporter._local_subset(taus)
    assert len(local) == 5
    np_taus = [t.float().cpu().numpy() for t in local]
    stats = X.head_stats(np_taus)
    heads = [(l, h) for l in range(5) for h in range(4)
             if X.classify(*stats[l, h, [0, 1, 2, 3]], 8) in ("long_range", "mid_range")]
    agg = X.aggregate(np_taus, np.ones((5, 4), bool) if not heads else
                      np.isin(np.arange(20).reshape(5, 4), [4 * l + h for l, h in heads]))
    vals = np.sort(agg[X.valid_mask(50, 8)])
    gaps = np.diff(vals)
    j = len(vals) // 2 + int(np.argmax(gaps[len(vals) // 2:len(vals) // 2 + 40]))
    thr = float((vals[j] + vals[j + 1]) / 2)  # a threshold away from every value
    tok = Tok()
    g_ref = E.UniversalLivingGraph()
    rg, rm, n_ref = reference_ingest(g_ref, ids[0].tolist(), np_taus, tok, thr, heads)
    g = E.UniversalLivingGraph()
    exp = E.TauExporter(g, edge_threshold=thr)
    st = exp.ingest(ids[0].tolist(), taus, tok)
    print(f"[export] heads={len(heads)} edges={st.edges_emitted} gini={st.concentration:.4f}", flush=True)
    assert st.edges_emitted == n_ref > 0
    assert st.signal_heads == (len(heads) or 20) and st.total_heads == 20
    assert st.used_head_fallback == (not heads)
    assert st.candidate_pairs == int(X.valid_mask(50, 8).sum())
    assert abs(st.concentration - rg) < 1e-5 and abs(st.aggregated_mean - rm) < 1e-6
    a, b = g.to_dict(), g_ref.to_dict()
    assert list(a["nodes"]) == list(b["nodes"])
    for k in a["nodes"]:
        na, nb = a["nodes"][k], b["nodes"][k]
        assert abs(na["activation"] - nb["activation"]) < 1e-6 and na["metadata"] == nb["metadata"]
    assert [(e["src"], e["dst"], e["metadata"]) for e in a["edges"]] == \
           [(e["src"], e["dst"], e["metadata"]) for e in b["edges"]]
    assert np.allclose([e["weight"] for e in a["edges"]], [e["weight"] for e in b["edges"]], atol=1e-6)


@pytest.mark.parametrize("use_triton", [False, True])
def test_streaming_step_rows_from_decode(dev, use_triton):
    """ingest_step on the cached decode step's rows (return_all mode) equals
    ingest_step on the full return_all forward's last rows (the reference's
    streaming loop, ts_bridge/streaming.py:26-33).  Six layers with global
    layers 2 and 5 in the middle and at the end; locked heads on either side
    of them and on a global layer, so a shifted layer index would show.
    With use_triton the plain forward normalises by the valid count, the
    return_all forward by tau mass: the cache must follow the latter."""
    from bozo_amd import model as M
    from bozo_amd.generation import TensionKVCache
    cfg = M.TensionConfig(vocab_size=60, dim=64, num_layers=6, num_heads=4, window=8, max_seq_len=64,
                          dropout=0.0, global_every=3, use_rope=True, use_triton=use_triton)
    torch.manual_seed(1)
    m = M.TensionLM(cfg).to(dev).eval()
    ids = torch.randint(0, 60, (1, 30), generator=torch.Generator().manual_seed(2)).to(dev)
    cache = TensionKVCache(m, 1, return_all=True)
    tok = Tok()
    heads = [(0, 1), (2, 3), (3, 2), (4, 0), (5, 1)]
    with torch.no_grad():
        logits, ptaus = cache.prefill(ids[:, :20])
        flg, _, ftaus = m(ids[:, :20], return_all=True)
        assert torch.equal(logits, flg)
        assert len(ptaus) == 6 and all(torch.equal(a, b) for a, b in zip(ptaus, ftaus))
        for t in range(20, 30):
            lg, rows = cache.step(ids[:, t], return_tau=True)
            flg, _, full = m(ids[:, :t + 1], return_all=True)
            assert len(rows) == 6 and all(r is not None for r in rows)
            assert (lg - flg[:, -1]).abs().max().item() <= 1e-4 * flg.abs().max().item()
            for i, (r, f) in enumerate(zip(rows, full)):
                assert r.shape == f[:, -1].shape, i
                assert (r - f[:, -1]).abs().max().item() < 1e-5, (t, i)
            ga, gb = E.UniversalLivingGraph(), E.UniversalLivingGraph()
            sa = E.StreamingTauExporter(ga, edge_threshold=0.0, head_override=heads)
            sb = E.StreamingTauExporter(gb, edge_threshold=0.0, head_override=heads)
            na = sa.ingest_step(ids[0, :t + 1].tolist(), rows, tok, query_abs_pos=t)
            nb = sb.ingest_step(ids[0, :t + 1].tolist(), full, tok, query_abs_pos=t)
            assert na == nb == 8
            wa = [e.weight for e in ga.edges]
            wb = [e.weight for e in gb.edges]
            assert np.allclose(wa, wb, atol=1e-5)
            assert [e.src for e in ga.edges] == [e.src for e in gb.edges]
    # rows of a plain cache carry None for the global layers: refused
    plain = TensionKVCache(m, 1)
    with torch.no_grad():
        plain.prefill(ids[:, :20])
        _, rows = plain.step(ids[:, 20], return_tau=True)
    assert rows[2] is None
    with pytest.raises(ValueError):
        E.StreamingTauExporter(E.UniversalLivingGraph(), edge_threshold=0.0).ingest_step(
            ids[0, :21].tolist(), rows, tok, query_abs_pos=20)
