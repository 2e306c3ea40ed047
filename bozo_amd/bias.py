"""Graph -> tau-bias builder with the per-pair lookups on the GPU.

Drop-in for the reference's ``ts_bridge/bias.py`` (``GraphBias``,
``BiasStats``): the content-pair -> weight map (edges collapsed by node
content, max weight, one relation) is built on the host as there
(``from_graph``), then copied once per device into an open-addressing hash
table (``tension_bias_table_insert``); ``local_bias`` / ``global_bias`` map
the context tokens to content ids on the host (T dictionary lookups) and one
kernel (``tension_bias_build``) writes the whole [B, T, W] / [B, T, T] bias
with its statistics, replacing the reference's O(T W) / O(T^2) Python loops.
The result feeds the tension kernels' ``bias`` argument directly.

Same arguments, results and semantics as the reference, including
``device="cpu"`` (the bias is built on the current GPU and copied back).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import numpy as np
import torch
from torch import Tensor

from . import _lib as L


def _content_of(node_id: str) -> str:
    """Strip a ``#pos`` suffix (bias.py:57-60)."""
    pos = node_id.rfind("#")
    return node_id if pos < 0 else node_id[:pos]


@dataclass
class BiasStats:
    nonzero_pairs: int = 0
    max_weight: float = 0.0
    mean_weight: float = 0.0


class GraphBias:
    """Content-addressed edge map and bias builder (bias.py:72-233)."""

    def __init__(self, edge_map: dict, alpha: float):
        self.edge_map = edge_map
        self.alpha = alpha
        self._tables: dict = {}

    @classmethod
    def from_graph(cls, graph, alpha: float = 0.5, relation: str = "tension") -> "GraphBias":
        edge_map: dict = {}
        for e in graph.edges:
            if e.relation != relation:
                continue
            key = (_content_of(e.src), _content_of(e.dst))
            if e.weight > edge_map.get(key, 0.0):
                edge_map[key] = e.weight
        return cls(edge_map=edge_map, alpha=alpha)

    def lookup(self, src_content: str, dst_content: str) -> float:
        return self.edge_map.get((src_content, dst_content), 0.0)

    def invalidate(self) -> None:
        """Drop the device tables (they are also rebuilt by themselves
        whenever ``edge_map`` differs from the map they were built from)."""
        self._tables.clear()

    # ---------------------------------------------------------------- device table

    def _table(self, dev: torch.device):
        # edge_map is a plain dict the caller may change in place (the
        # reference exposes it so): the table is reused only while the map
        # equals the copy it was built from (~2 ms for 50 K edges)
        hit = self._tables.get(dev)
        if hit is not None and hit[0] == self.edge_map:
            return hit[1]
        snap = dict(self.edge_map)
        cid: dict = {}
        for (s, d) in self.edge_map:
            cid.setdefault(s, len(cid))
            cid.setdefault(d, len(cid))
        n = len(self.edge_map)
        log2cap = max(1, int(np.ceil(np.log2(max(2 * n, 2)))))
        keys = torch.full((1 << log2cap,), -1, dtype=torch.int64, device=dev)
        vals = torch.zeros(1 << log2cap, dtype=torch.float64, device=dev)
        if n:
            pairs = np.array([(cid[s], cid[d]) for (s, d) in self.edge_map], dtype=np.uint64)
            kin = torch.from_numpy(((pairs[:, 0] << np.uint64(32)) | pairs[:, 1]).view(np.int64)).to(dev)
            vin = torch.tensor(list(self.edge_map.values()), dtype=torch.float64, device=dev)
            with torch.cuda.device(dev):
                L.check(L.lib().tension_bias_table_insert(
                    kin.data_ptr(), vin.data_ptr(), n, keys.data_ptr(), vals.data_ptr(), log2cap,
                    torch.cuda.current_stream(dev).cuda_stream), "tension_bias_table_insert")
        table = (cid, keys, vals, log2cap)
        self._tables[dev] = (snap, table)
        return table

    def _build(self, ctx_ids, tokenizer, W: int, batch: int, device, dtype):
        if not torch.cuda.is_available():
            raise RuntimeError("the bias builder runs on the GPU; no GPU is available")
        want = torch.device(device)
        dev = want if want.type == "cuda" else torch.device("cuda", torch.cuda.current_device())
        if dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        cid, keys, vals, log2cap = self._table(dev)
        T = len(ctx_ids)
        contents = [tokenizer.id_to_token(int(t)) or f"<{int(t)}>" for t in ctx_ids]
        ids = torch.tensor([cid.get(c, -1) for c in contents], dtype=torch.int32).to(dev)
        K = W if W > 0 else T
        bias = torch.empty((batch, T, K), dtype=dtype, device=dev)
        stats = torch.zeros(3, dtype=torch.float64, device=dev)
        with torch.cuda.device(dev):
            L.check(L.lib().tension_bias_build(
                ids.data_ptr(), batch, T, W, keys.data_ptr(), vals.data_ptr(), log2cap,
                float(self.alpha), L.buf(bias), stats.data_ptr(),
                torch.cuda.current_stream(dev).cuda_stream), "tension_bias_build")
        hits, total, mx = stats.tolist()
        st = BiasStats(nonzero_pairs=int(hits), max_weight=mx, mean_weight=total / hits if hits else 0.0)
        return (bias if want.type == "cuda" else bias.to(want)), st

    def local_bias(self, ctx_ids: Sequence[int], tokenizer, window: int, batch: int = 1,
                   device="cpu", dtype: torch.dtype = torch.float32):
        """[B, T, W] bias, bias[b, t, w] = alpha * weight(ctx[t - (W - w)] ->
        ctx[t]), zero where that key is before the context (bias.py:141-187)."""
        if window < 1:
            raise ValueError("window must be >= 1")
        return self._build(ctx_ids, tokenizer, int(window), batch, device, dtype)

    def global_bias(self, ctx_ids: Sequence[int], tokenizer, batch: int = 1, device="cpu",
                    dtype: torch.dtype = torch.float32):
        """[B, T, T] bias, bias[b, t, s] = alpha * weight(ctx[s] -> ctx[t]) for
        s < t, zero otherwise (bias.py:189-233)."""
        return self._build(ctx_ids, tokenizer, 0, batch, device, dtype)
