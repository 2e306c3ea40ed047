"""Tau export to a constraint graph, with the reductions on the GPU.

Drop-in for the reference's ``ts_bridge`` exporter (``export.py``,
``head_filter.py``, ``streaming.py``) and its graph container
(``graph.py``; same node/edge fields and JSON layout).  The reference copies
every layer's tau [B,T,H,W] to the host and reduces it with numpy; here the
per-head statistics (``tension_tau_head_stats``) and the head-masked
aggregate (``tension_tau_aggregate``) run on the device over the tau the
kernels materialised, the Gini / mean / edge selection reduce the [T, W]
aggregate on the device, and only the emitted edges (plus one pull value per
query) cross to the host to be written into the graph.

Same public names, arguments and results as the reference: ``HeadRole``,
``HeadStat``, ``profile_heads``, ``select_signal_heads``, ``ExportStats``,
``TauExporter`` (``profile_and_lock``, ``ingest``),
``StreamingTauExporter`` (``prime``, ``ingest_step``) and
``UniversalLivingGraph``.  ``ingest_step`` also takes the [B, H, W] tau rows
the cached decode step returns (``TensionKVCache.step(return_tau=True)``)
in place of full [B, T, H, W] tensors.
"""
from __future__ import annotations

import json
from dataclasses import asdict, dataclass, field
from enum import Enum
from pathlib import Path
from typing import Iterable, Optional, Sequence

import torch
from torch import Tensor

from . import _lib as L

_MAX_TAU_FLOOR = 0.40   # head_filter.py:68-69
_CONCENTRATION = 0.35


class HeadRole(str, Enum):
    INACTIVE = "inactive"
    SYNTACTIC = "syntactic"
    LONG_RANGE = "long_range"
    DIFFUSE = "diffuse"
    MID_RANGE = "mid_range"


@dataclass
class HeadStat:
    layer: int
    head: int
    mean_tau: float
    max_tau: float        # 0.99 quantile
    peak_pos: float       # mean first arg-max over the window
    concentration: float  # mean max over the window
    role: HeadRole

    @property
    def carries_graph_signal(self) -> bool:
        return self.role in (HeadRole.LONG_RANGE, HeadRole.MID_RANGE)


def _classify(max_tau: float, peak_pos: float, concentration: float, W: int) -> HeadRole:
    """head_filter.py:74-90."""
    if max_tau < _MAX_TAU_FLOOR:
        return HeadRole.INACTIVE
    if concentration < _CONCENTRATION:
        return HeadRole.DIFFUSE
    if peak_pos > W * 0.7:
        return HeadRole.SYNTACTIC
    if peak_pos < W * 0.3:
        return HeadRole.LONG_RANGE
    return HeadRole.MID_RANGE


# ------------------------------------------------------------------ device reductions

def _taus_arg(taus: Sequence[Tensor]):
    if not taus:
        raise ValueError("no tau tensors")
    if len(taus) > 32:
        raise ValueError(f"at most 32 layers per call, got {len(taus)}")
    shape = tuple(taus[0].shape)
    for t in taus:
        if t.dim() != 4 or tuple(t.shape) != shape:
            raise ValueError("every tau must be [B, T, H, W] of one shape")
        if not t.is_cuda:
            raise RuntimeError("tau export runs on the GPU; got a CPU tensor")
        if t.device != taus[0].device:
            raise ValueError(f"every tau must be on {taus[0].device}, got one on {t.device}")
    rows = [t if t.stride(-1) == 1 else t.contiguous() for t in taus]
    arr = (L.TensionBuf * len(rows))(*[L.buf(t).contents for t in rows])
    return arr, rows, shape


def head_stats(taus: Sequence[Tensor], valid_only: bool = False) -> Tensor:
    """Per (layer, head) statistics of the batch-mean tau: float32 [L, H, 4]
    on the device = mean, 0.99 quantile, mean first arg-max over w, mean max
    over w (head_filter.py:98-130; ``valid_only`` zeroes cells t + w < W
    first, corpus_profile.py:58-98)."""
    arr, rows, (B, T, H, W) = _taus_arg(taus)
    dev = rows[0].device
    out = torch.empty(len(rows), H, 4, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        L.check(L.lib().tension_tau_head_stats(
            arr, len(rows), B, T, H, W, out.data_ptr(), L.TAU_VALID_ONLY if valid_only else 0,
            torch.cuda.current_stream(dev).cuda_stream), "tension_tau_head_stats")
    return out


def aggregate_tau(taus: Sequence[Tensor], head_mask: Tensor) -> Tensor:
    """aggregated[t, w] = mean over the selected (layer, head) pairs of the
    batch-mean tau (export.py:185-200); all pairs when none is selected.
    head_mask: bool [L, H]."""
    arr, rows, (B, T, H, W) = _taus_arg(taus)
    dev = rows[0].device
    mask = head_mask.to(device=dev, dtype=torch.int32).contiguous()
    if tuple(mask.shape) != (len(rows), H):
        raise ValueError(f"head_mask must be [{len(rows)}, {H}]")
    out = torch.empty(T, W, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        L.check(L.lib().tension_tau_aggregate(
            arr, len(rows), B, T, H, W, mask.data_ptr(), out.data_ptr(),
            torch.cuda.current_stream(dev).cuda_stream), "tension_tau_aggregate")
    return out


def _valid(T: int, W: int, dev) -> Tensor:
    return (torch.arange(T, device=dev)[:, None] + torch.arange(W, device=dev)[None, :]) >= W


def concentration(agg: Tensor) -> tuple:
    """(Gini, mean) of the aggregate over its valid pairs (export.py:202-218)."""
    T, W = agg.shape
    vals = agg[_valid(T, W, agg.device)].double()
    n = vals.numel()
    if n == 0:
        return 0.0, 0.0
    total = vals.sum()
    mean = float(total / n)
    if n > 1 and float(total) > 1e-9:
        cum = torch.cumsum(torch.sort(vals).values, 0)
        return float((n + 1 - 2 * cum.sum() / cum[-1]) / n), mean
    return 0.0, mean


def profile_heads(all_tensions: list) -> list:
    """head_filter.py:98-130, statistics on the device."""
    st = head_stats(all_tensions).cpu().tolist()
    W = int(all_tensions[0].shape[-1])
    out = []
    for l, layer in enumerate(st):
        for h, (mean_t, max_t, peak, conc) in enumerate(layer):
            out.append(HeadStat(l, h, mean_t, max_t, peak, conc, _classify(max_t, peak, conc, W)))
    return out


def select_signal_heads(stats: Iterable[HeadStat], include_mid_range: bool = True) -> list:
    allowed = {HeadRole.LONG_RANGE}
    if include_mid_range:
        allowed.add(HeadRole.MID_RANGE)
    return [(s.layer, s.head) for s in stats if s.role in allowed]


# ------------------------------------------------------------------ graph container

@dataclass
class Node:
    id: str
    content: str
    topics: list = field(default_factory=list)
    activation: float = 0.5
    stability: float = 0.5
    base_strength: float = 0.5
    metadata: dict = field(default_factory=dict)


@dataclass
class Edge:
    src: str
    dst: str
    weight: float
    relation: str = "tension"
    metadata: dict = field(default_factory=dict)


class UniversalLivingGraph:
    """Node/edge container with the reference's fields, reinforcement rules
    and JSON layout (graph.py:37-184).  Edges are indexed by (src, dst,
    relation), so reinforcing one is O(1) instead of a scan of the edge list;
    insertion order is kept."""

    def __init__(self):
        self.nodes: dict = {}
        self.edges: list = []
        self._eidx: dict = {}

    def upsert_node(self, id, content, activation=None, stability=None, base_strength=None,
                    topics=None, metadata=None):
        node = self.nodes.get(id)
        if node is None:
            node = Node(id=id, content=content, topics=topics or [],
                        activation=0.5 if activation is None else activation,
                        stability=0.5 if stability is None else stability,
                        base_strength=0.5 if base_strength is None else base_strength,
                        metadata=metadata or {})
            self.nodes[id] = node
            return node
        if activation is not None:
            node.activation = max(node.activation, activation)
        if stability is not None:
            node.stability = max(node.stability, stability)
        if base_strength is not None:
            node.base_strength = max(node.base_strength, base_strength)
        if topics:
            node.topics = sorted(set(node.topics) | set(topics))
        if metadata:
            node.metadata.update(metadata)
        return node

    def add_edge(self, src, dst, weight, relation="tension", metadata=None):
        key = (src, dst, relation)
        e = self._eidx.get(key)
        if e is not None:
            if weight > e.weight:
                e.weight = weight
            if metadata:
                e.metadata.update(metadata)
            return e
        e = Edge(src=src, dst=dst, weight=weight, relation=relation, metadata=metadata or {})
        self.edges.append(e)
        self._eidx[key] = e
        return e

    def density(self) -> float:
        n = len(self.nodes)
        return 0.0 if n < 2 else len(self.edges) / (n * (n - 1) / 2)

    def mean_activation(self) -> float:
        return sum(n.activation for n in self.nodes.values()) / len(self.nodes) if self.nodes else 0.0

    def mean_edge_weight(self) -> float:
        return sum(e.weight for e in self.edges) / len(self.edges) if self.edges else 0.0

    def to_dict(self) -> dict:
        return {"nodes": {i: asdict(n) for i, n in self.nodes.items()},
                "edges": [asdict(e) for e in self.edges]}

    def to_json(self, path) -> None:
        Path(path).write_text(json.dumps(self.to_dict(), indent=2))

    @classmethod
    def from_dict(cls, data: dict) -> "UniversalLivingGraph":
        g = cls()
        for i, n in data.get("nodes", {}).items():
            g.nodes[i] = Node(**n)
        for e in data.get("edges", []):
            edge = Edge(**e)
            g.edges.append(edge)
            g._eidx.setdefault((edge.src, edge.dst, edge.relation), edge)
        return g

    @classmethod
    def from_json(cls, path) -> "UniversalLivingGraph":
        return cls.from_dict(json.loads(Path(path).read_text()))

    def __repr__(self) -> str:
        return (f"UniversalLivingGraph(nodes={len(self.nodes)}, edges={len(self.edges)}, "
                f"density={self.density():.3f}, mean_act={self.mean_activation():.3f})")


# ------------------------------------------------------------------ exporter

@dataclass
class ExportStats:
    tokens: int
    signal_heads: int
    total_heads: int
    candidate_pairs: int
    edges_emitted: int
    nodes_touched: int
    mean_weight: float
    concentration: float = 0.0
    aggregated_mean: float = 0.0
    used_head_fallback: bool = False


def _tok(tokenizer, i: int) -> str:
    return tokenizer.id_to_token(i) or f"<{i}>"


class TauExporter:
    """Writes aggregated tau as weighted edges key -> query into a graph
    (export.py:67-302)."""

    def __init__(self, graph, edge_threshold: float = 0.3, include_mid_range: bool = True,
                 head_override: Optional[list] = None, position_scoped_ids: bool = True):
        self.graph = graph
        self.edge_threshold = edge_threshold
        self.include_mid_range = include_mid_range
        self.position_scoped_ids = position_scoped_ids
        self._locked_heads = head_override

    @staticmethod
    def _local_subset(all_tensions: list) -> list:
        """Layers with the most common (H, W) (export.py:93-104)."""
        shapes = [tuple(t.shape[-2:]) for t in all_tensions]
        canonical = max(set(shapes), key=shapes.count)
        return [t for t in all_tensions if tuple(t.shape[-2:]) == canonical]

    def profile_and_lock(self, all_tensions: list) -> list:
        stats = profile_heads(self._local_subset(all_tensions))
        self._locked_heads = select_signal_heads(stats, include_mid_range=self.include_mid_range)
        return stats

    def reset_head_lock(self) -> None:
        self._locked_heads = None

    def _current_signal_heads(self, local: list) -> list:
        if self._locked_heads is not None:
            return self._locked_heads
        return select_signal_heads(profile_heads(local), include_mid_range=self.include_mid_range)

    def _node_id(self, tok: str, pos: int) -> str:
        return f"{tok}#{pos}" if self.position_scoped_ids else tok

    def ingest(self, token_ids: Sequence[int], all_tensions: list, tokenizer,
               position_offset: int = 0) -> ExportStats:
        T = len(token_ids)
        if not all_tensions:
            return ExportStats(tokens=T, signal_heads=0, total_heads=0, candidate_pairs=0,
                               edges_emitted=0, nodes_touched=0, mean_weight=0.0)
        local = self._local_subset(all_tensions)
        Ln = len(local)
        H, W = (int(x) for x in local[0].shape[-2:])
        local = [t.detach()[:, :T] for t in local]
        heads = self._current_signal_heads(local)
        mask = torch.zeros(Ln, H, dtype=torch.bool)
        fallback = not heads
        if fallback:
            mask[:] = True
        else:
            for (l, h) in heads:
                mask[l, h] = True
        agg = aggregate_tau(local, mask)                       # [T, W] on the device
        gini, agg_mean = concentration(agg)
        valid = _valid(T, W, agg.device)
        emit = valid & (agg >= self.edge_threshold)
        tw = torch.nonzero(emit).cpu().tolist()
        weights = agg[emit].cpu().tolist()
        pull = agg.mean(-1).cpu().tolist()

        g = self.graph
        touched = set()
        e = 0
        for t in range(T):
            q_abs = t + position_offset
            q_tok = _tok(tokenizer, token_ids[t])
            qid = self._node_id(q_tok, q_abs)
            g.upsert_node(id=qid, content=q_tok, activation=min(1.0, 0.3 + pull[t]),
                          metadata={"absolute_pos": q_abs, "token_id": int(token_ids[t])})
            touched.add(qid)
            while e < len(tw) and tw[e][0] == t:
                w = tw[e][1]
                s = t - (W - w)
                wt = weights[e]
                k_abs = s + position_offset
                k_tok = _tok(tokenizer, token_ids[s])
                kid = self._node_id(k_tok, k_abs)
                g.upsert_node(id=kid, content=k_tok, activation=min(1.0, 0.3 + wt),
                              metadata={"absolute_pos": k_abs, "token_id": int(token_ids[s])})
                touched.add(kid)
                g.add_edge(src=kid, dst=qid, weight=wt, relation="tension",
                           metadata={"distance": t - s})
                e += 1
        candidates = sum(min(t, W) for t in range(T))  # pairs with s = t - (W - w) >= 0
        return ExportStats(tokens=T, signal_heads=int(mask.sum()), total_heads=Ln * H,
                           candidate_pairs=candidates, edges_emitted=len(tw),
                           nodes_touched=len(touched),
                           mean_weight=float(sum(weights) / len(weights)) if weights else 0.0,
                           concentration=gini, aggregated_mean=agg_mean,
                           used_head_fallback=fallback)


class StreamingTauExporter(TauExporter):
    """Prime on the prompt, then emit the edges of one new query per step
    (streaming.py:53-202)."""

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        self._touched_nodes: set = set()
        self._stream_steps = 0
        self._stream_edges = 0

    def prime(self, prompt_ids, all_tensions: list, tokenizer, position_offset: int = 0):
        if self._locked_heads is None:
            self.profile_and_lock(all_tensions)
        stats = self.ingest(prompt_ids, all_tensions, tokenizer, position_offset=position_offset)
        self._touched_nodes.update(self.graph.nodes.keys())
        return stats

    def ingest_step(self, ctx_ids, all_tensions: list, tokenizer, query_abs_pos: int) -> int:
        """Edges from the last query of ``ctx_ids`` to its W keys.  Each
        entry of ``all_tensions`` is a layer's [B,T,H,W] tau (its last row is
        used) or the [B,H,W] row of a cached decode step, one entry per layer
        as ``model(ctx, return_all=True)`` lists them: the locked (layer,
        head) pairs index that list (after the most-common-shape rule), so a
        missing layer would shift them.  Decode rows come from
        ``TensionKVCache(model, N, return_all=True).step(ids,
        return_tau=True)``, which includes the global layers' rows."""
        if any(t is None for t in all_tensions):
            raise ValueError(
                "ingest_step needs a tau row for every layer (None given): use the rows of "
                "TensionKVCache(model, N, return_all=True).step(..., return_tau=True)")
        rows = [t if t.dim() == 3 else t[:, -1] for t in all_tensions]
        if not rows or not ctx_ids:
            return 0
        local = self._local_subset(rows)
        Ln = len(local)
        H, W = (int(x) for x in local[0].shape[-2:])
        mask = torch.zeros(Ln, H, dtype=torch.bool)
        if self._locked_heads:
            for (l, h) in self._locked_heads:
                if 0 <= l < Ln and 0 <= h < H:
                    mask[l, h] = True
        if not mask.any():
            mask[:] = True
        agg = aggregate_tau([t.detach()[:, None] for t in local], mask)[0]   # [W]
        vals = agg.cpu().tolist()

        T_ctx = len(ctx_ids)
        q_int = int(ctx_ids[-1])
        q_tok = _tok(tokenizer, q_int)
        qid = self._node_id(q_tok, query_abs_pos)
        self.graph.upsert_node(id=qid, content=q_tok, activation=min(1.0, 0.3 + sum(vals) / W),
                               metadata={"absolute_pos": query_abs_pos, "token_id": q_int})
        self._touched_nodes.add(qid)
        emitted = 0
        for w in range(W):
            back = W - w
            idx = T_ctx - 1 - back
            if idx < 0 or vals[w] < self.edge_threshold:
                continue
            k_abs = query_abs_pos - back
            k_int = int(ctx_ids[idx])
            k_tok = _tok(tokenizer, k_int)
            kid = self._node_id(k_tok, k_abs)
            self.graph.upsert_node(id=kid, content=k_tok, activation=min(1.0, 0.3 + vals[w]),
                                   metadata={"absolute_pos": k_abs, "token_id": k_int})
            self._touched_nodes.add(kid)
            self.graph.add_edge(src=kid, dst=qid, weight=vals[w], relation="tension",
                                metadata={"distance": back})
            emitted += 1
        self._stream_steps += 1
        self._stream_edges += emitted
        return emitted
