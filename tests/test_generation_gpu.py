"""KV-cached generation (bozo_amd/generation.py) against the full forward.

The reference generates by re-running the forward over the context for every
token (model.py:617-652,719-768); the cached step must give the same logits
as that forward's last row, layer caches filled by a prefill.  The float32
steps are checked against the float64 functional restatement of the
reference forward (oracle/model_ref.py) and against the HIP model's own
full forward.  Checked per
step on float32 models (exact decode kernel, 1e-5 relative) and bf16
autocast at head_dim 64 (the fast decode kernel, including a global layer
window of max_seq_len slots, 2e-2 relative), plus the sampled token
sequence of ``generate_cached`` against the reference's re-forward loop with
the same sampler and seed, across the point where the context starts to
slide.
"""
import numpy as np
import pytest
import torch

from bozo_amd import model as M
from bozo_amd.generation import TensionKVCache, generate_cached, sample_next
from oracle import model_ref
from tests._util import rel_l2

pytestmark = pytest.mark.gpu


def make_model(cfg, seed, dev):
    torch.manual_seed(seed)
    m = M.TensionLM(cfg)
    with torch.no_grad():
        for p in m.parameters():
            p.add_(0.05 * torch.randn_like(p))
    return m.to(dev).eval()


@pytest.mark.parametrize("use_rope,use_triton", [(True, True), (True, False), (False, True)])
def test_cached_steps_match_full_forward_f32(dev, use_rope, use_triton):
    cfg = M.TensionConfig(vocab_size=80, dim=64, num_layers=4, num_heads=4, window=6,
                          max_seq_len=40, dropout=0.0, global_every=2, use_rope=use_rope,
                          use_triton=use_triton)
    m = make_model(cfg, 3, dev)
    g = torch.Generator().manual_seed(8)
    N, P, L = 2, 9, 40
    ids = torch.randint(0, cfg.vocab_size, (N, L), generator=g).to(dev)
    print(f"[gen f32] rope={use_rope} triton={use_triton}", flush=True)
    cache = TensionKVCache(m, N)
    with torch.no_grad():
        pre = cache.prefill(ids[:, :P])
        assert rel_l2(pre.cpu().numpy(), m(ids[:, :P]).cpu().numpy()) == 0.0
        for t in range(P, L):
            got, taus = cache.step(ids[:, t], return_tau=True)
            full, _, ftaus = m(ids[:, :t + 1], return_all=True)
            ref = m(ids[:, :t + 1])[:, -1]  # the reference's generation forward
            assert rel_l2(got.cpu().numpy(), ref.cpu().numpy()) < 1e-5, t
            # return_all switches the Triton-path local layers to tau-mass
            # normalisation (model.py:250-258), so past layer 0 the taus of
            # that forward match the cached (count-normalised) step only
            # when use_triton is off
            for i, (blk, a, b) in enumerate(zip(m.blocks, taus, ftaus)):
                if blk.global_layer:
                    assert a is None
                elif i == 0 or not use_triton:
                    assert np.max(np.abs(a.cpu().numpy() - b[:, -1].cpu().numpy())) < 1e-5
    assert cache.t == L
    with pytest.raises(ValueError):
        cache.step(ids[:, 0])


@pytest.mark.parametrize("use_rope,use_triton", [(True, True), (True, False), (False, True)])
def test_cached_steps_match_oracle_f64(dev, use_rope, use_triton):
    """Prefill and every cached step (float32 model, exact decode kernel)
    against the functional float64 restatement of the reference forward
    (oracle/model_ref.py, same state_dict) over the whole context, last row:
    what the reference's generation loop computes per token
    (model.py:617-652,719-768).  W = 6 and 31 steps past a 9-token prompt,
    so every local ring wraps several times; the global layers' caches fill
    to max_seq_len."""
    cfg = M.TensionConfig(vocab_size=80, dim=64, num_layers=4, num_heads=4, window=6,
                          max_seq_len=40, dropout=0.0, global_every=2, use_rope=use_rope,
                          use_triton=use_triton)
    m = make_model(cfg, 13, dev)
    sd = {k: v.detach().double().cpu() for k, v in m.state_dict().items()}
    g = torch.Generator().manual_seed(15)
    N, P, L = 2, 9, 40
    ids = torch.randint(0, cfg.vocab_size, (N, L), generator=g)
    print(f"[gen oracle] rope={use_rope} triton={use_triton}", flush=True)
    cache = TensionKVCache(m, N)
    worst = 0.0
    with torch.no_grad():
        pre = cache.prefill(ids[:, :P].to(dev)).double().cpu().numpy()
        ref = model_ref.forward(sd, cfg, ids[:, :P]).numpy()
        err = rel_l2(pre, ref)
        assert err < 1e-5, ("prefill", err)
        for t in range(P, L):
            got = cache.step(ids[:, t].to(dev)).double().cpu().numpy()
            ref = model_ref.forward(sd, cfg, ids[:, :t + 1])[:, -1].numpy()
            err = rel_l2(got, ref)
            worst = max(worst, err)
            assert err < 1e-5, (t, err)
    print(f"  worst step rel L2 {worst:.2e}", flush=True)


@pytest.mark.parametrize("use_triton", [True, False])
def test_cached_steps_match_full_forward_bf16(dev, use_triton):
    cfg = M.TensionConfig(vocab_size=512, dim=128, num_layers=4, num_heads=2, window=64,
                          max_seq_len=320, dropout=0.0, global_every=2, use_rope=True,
                          use_triton=use_triton)
    m = make_model(cfg, 4, dev)
    g = torch.Generator().manual_seed(9)
    N, P, S = 3, 250, 12
    ids = torch.randint(0, cfg.vocab_size, (N, P + S), generator=g).to(dev)
    print(f"[gen bf16] triton={use_triton}", flush=True)
    cache = TensionKVCache(m, N)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        cache.prefill(ids[:, :P])
        for t in range(P, P + S):
            got = cache.step(ids[:, t]).float()
            ref = m(ids[:, :t + 1])[:, -1].float()
            err = rel_l2(got.cpu().numpy(), ref.cpu().numpy())
            assert err < 2e-2, (t, err)


@pytest.mark.parametrize("bf16", [False, True])
def test_graph_step_matches_eager(dev, bf16):
    """Every replay of the captured step equals the eager step (two caches
    from the same prefill, eager work between the replays)."""
    cfg = M.TensionConfig(vocab_size=256, dim=128, num_layers=4, num_heads=2, window=16,
                          max_seq_len=96, dropout=0.0, global_every=2, use_rope=True,
                          use_triton=True)
    m = make_model(cfg, 6, dev)
    N, P, S = 2, 30, 20
    ids = torch.randint(0, cfg.vocab_size, (N, P + S), generator=torch.Generator().manual_seed(12)).to(dev)
    print(f"[gen graph] bf16={bf16}", flush=True)
    ctx = torch.autocast("cuda", dtype=torch.bfloat16) if bf16 else torch.autocast("cuda", enabled=False)
    with torch.no_grad(), ctx:
        ea, gr = TensionKVCache(m, N), TensionKVCache(m, N)
        ea.prefill(ids[:, :P])
        gr.prefill(ids[:, :P])
        for t in range(P, P + S):
            a = ea.step(ids[:, t]).float()
            b = gr.graph_step(ids[:, t]).float().clone()
            torch.cuda.synchronize()
            assert torch.allclose(a, b, rtol=1e-5, atol=1e-5), (t, (a - b).abs().max().item())
    for ca, cb in zip(ea.layers, gr.layers):
        assert torch.equal(ca.k, cb.k) and torch.equal(ca.v, cb.v)
        assert torch.equal(ca.pos[ca.cur], cb.pos[cb.cur])


def reforward_generate(model, input_ids, max_new, temp, top_p, rep_penalty, generator):
    """The reference's generation loop (model.py:625-652) with the same sampler."""
    dev = next(model.parameters()).device
    ids = list(input_ids)
    for _ in range(max_new):
        ctx = torch.tensor([ids[-model.cfg.max_seq_len:]], dtype=torch.long, device=dev)
        with torch.no_grad():
            logits = model(ctx)[0, -1]
        ids.append(sample_next(logits, ids, temp, top_p, rep_penalty, generator))
    return ids


def test_generate_cached_matches_reforward(dev):
    cfg = M.TensionConfig(vocab_size=64, dim=64, num_layers=4, num_heads=4, window=8,
                          max_seq_len=48, dropout=0.1, global_every=2, use_rope=True,
                          use_triton=True)
    m = make_model(cfg, 5, dev)
    prompt = torch.randint(0, cfg.vocab_size, (20,), generator=torch.Generator().manual_seed(10)).tolist()
    b = reforward_generate(m, prompt, 40, 0.9, 0.95, 1.3, torch.Generator(device=dev).manual_seed(11))
    for use_graph in (False, True):
        a = generate_cached(m, prompt, max_new=40, temp=0.9, top_p=0.95, rep_penalty=1.3,
                            generator=torch.Generator(device=dev).manual_seed(11), use_graph=use_graph)
        print(f"[gen sample] graph={use_graph} {a[20:30]}", flush=True)
        assert len(a) == 60 and a[:20] == prompt
        assert a == b
