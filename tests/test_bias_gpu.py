"""Graph-bias builder on the GPU (bozo_amd/bias.py) against the reference's
loops (oracle/bias_ref.py)."""
import numpy as np
import pytest
import torch

from bozo_amd.bias import GraphBias
from oracle import bias_ref as R

pytestmark = pytest.mark.gpu


class Tok:
    def id_to_token(self, i):
        return None if i % 11 == 5 else f"w{i % 97}"


def make(seed, n_contents, n_edges, T):
    r = np.random.default_rng(seed)
    names = [f"w{i}" for i in range(n_contents)] + [f"<{i}>" for i in range(5, 400, 11)]
    assert n_edges <= len(names) ** 2 // 2, "not that many distinct pairs"
    edge_map = {}
    while len(edge_map) < n_edges:
        a, b = r.choice(names, 2)
        edge_map[(str(a), str(b))] = float(r.random() * 1.2 - 0.2)  # some <= 0
    ids = r.integers(0, 400, T).tolist()
    return edge_map, ids


@pytest.mark.parametrize("n_edges,T,W,batch,dtype", [
    (50, 37, 8, 1, torch.float32), (3000, 300, 64, 2, torch.float32),
    (3000, 300, 64, 1, torch.bfloat16), (0, 20, 4, 1, torch.float32), (8000, 200, 16, 1, torch.float64)])
def test_local_bias_matches_reference(dev, n_edges, T, W, batch, dtype):
    edge_map, ids = make(n_edges + T, 97, n_edges, T)
    gb = GraphBias(edge_map, alpha=0.6)
    tok = Tok()
    bias, st = gb.local_bias(ids, tok, window=W, batch=batch, device=dev, dtype=dtype)
    contents = [tok.id_to_token(i) or f"<{i}>" for i in ids]
    ref, (hits, mx, mean) = R.local_bias(edge_map, 0.6, contents, W, batch, dtype=np.float64)
    ref_t = torch.from_numpy(ref)
    if dtype != torch.float64:
        ref_t = ref_t.float().to(dtype)
    assert bias.shape == (batch, T, W) and bias.dtype == dtype
    assert torch.equal(bias.cpu(), ref_t)
    assert st.nonzero_pairs == hits and st.max_weight == mx
    assert abs(st.mean_weight - mean) <= 1e-12 * max(1.0, mean)
    print(f"[bias local] edges={n_edges} T={T} W={W} hits={hits}", flush=True)


@pytest.mark.parametrize("T", [1, 65, 400])
def test_global_bias_matches_reference(dev, T):
    edge_map, ids = make(T, 97, 4000, T)
    gb = GraphBias(edge_map, alpha=1.5)
    tok = Tok()
    bias, st = gb.global_bias(ids, tok, batch=1, device="cpu")
    contents = [tok.id_to_token(i) or f"<{i}>" for i in ids]
    ref, (hits, mx, mean) = R.global_bias(edge_map, 1.5, contents)
    assert bias.device.type == "cpu" and bias.shape == (1, T, T)
    assert torch.equal(bias, torch.from_numpy(ref))
    assert st.nonzero_pairs == hits and st.max_weight == mx


def test_bias_feeds_the_model_and_table_refresh(dev):
    from bozo_amd import model as M
    cfg = M.TensionConfig(vocab_size=400, dim=64, num_layers=2, num_heads=4, window=8, max_seq_len=64,
                          dropout=0.0, global_every=2, use_rope=True, use_triton=True)
    torch.manual_seed(0)
    m = M.TensionLM(cfg).to(dev).eval()
    edge_map, ids = make(7, 97, 2000, 50)
    gb = GraphBias(edge_map, alpha=0.5)
    tok = Tok()
    lb, _ = gb.local_bias(ids, tok, window=8, device=dev)
    gbias, _ = gb.global_bias(ids, tok, device=dev)
    x = torch.tensor([ids], device=dev)
    with torch.no_grad():
        a = m(x)
        b = m(x, tau_bias=lb, tau_bias_global=gbias)
    assert torch.isfinite(b).all() and not torch.allclose(a, b)
    # a new edge after the first build is seen (the map's size changes)
    contents = [tok.id_to_token(i) or f"<{i}>" for i in ids]
    gb.edge_map[(contents[0], contents[1])] = 5.0
    lb2, st2 = gb.local_bias(ids, tok, window=8, device=dev)
    assert lb2[0, 1, 7].item() == pytest.approx(2.5)
    # in-place changes that keep the size: a new weight, and one key swapped
    # for another; each build equals the reference's lookup loop
    gb.edge_map[(contents[0], contents[1])] = 3.0
    lb3, _ = gb.local_bias(ids, tok, window=8, device=dev)
    assert lb3[0, 1, 7].item() == pytest.approx(1.5)
    del gb.edge_map[(contents[0], contents[1])]
    gb.edge_map[(contents[2], contents[3])] = 4.0
    lb4, _ = gb.local_bias(ids, tok, window=8, device=dev)
    got = lb4[0].cpu().numpy()
    for t in range(len(ids)):
        for w in range(8):
            s = t - (8 - w)
            wt = 0.0 if s < 0 else gb.lookup(contents[s], contents[t])
            assert got[t, w] == np.float32(0.5 * wt if wt > 0 else 0.0), (t, w)
