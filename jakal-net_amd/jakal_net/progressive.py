"""The Progressive-B query-block training step, composed from the hot-path operators.

This is the caller of the native path that BASELINE config 5 times: a token
prefix becomes a sequence layer S; window propagations warm it up; joint
blocks exchange information between S and two slot layers (an expanded layer
B_exp and a compressed layer B_cmp); a block of query slots, fed the
teacher-forced shifted targets, reads S through a transition and itself
through causal dense propagation; an MLP head scores the vocabulary.

The order of operators in a joint block follows the reference's
ProgressiveBJointBlock.forward (scripts/progressive_b_example.py:1108-1323):

    S       <- window propagation of S
    B_exp   <- transition B_cmp -> B_exp (expand), then top-k propagation of B_exp
    S       <- transition B_exp -> S
    B_cmp   <- transition B_exp -> B_cmp (compress), then S -> B_cmp,
               then top-k propagation of B_cmp

and the query path follows forward_query_block (:2059-2152): query slots
initialised from the shifted target embeddings (:2026-2047), then
`query_refine` rounds of transition S -> Q (:1957-1975) and causal dense
propagation over Q (:1977-2012), then the head.  Every operator is a
LowRankBilinearPairwise / LowRankBilinearRoute module, so with
implementation="native" each one runs on the HIP library.

The glue is this module's own (not the reference script's): every update
merges as  layer <- (tanh(state + a * delta_state), LayerNorm(val + a *
delta_val)),  with a fixed scale `a` per path; slot layers start from learned
templates; positions are a learned table.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor, nn
from torch.nn import functional as F

from jakal_net.core import Layer, LayerDelta
from jakal_net.modules import LowRankBilinearPairwise, LowRankBilinearRoute
from jakal_net.propagation import SparsePropagation
from jakal_net.transition import SparseTransition


@dataclass(frozen=True)
class ProgressiveBConfig:
    """Sizes of the step.  The defaults are BASELINE config 5."""

    vocab: int = 16384
    dim: int = 512
    prefix: int = 512          # sequence nodes (prefix tokens)
    query: int = 64            # query slots (predicted tokens)
    rank: int = 64             # low-rank score / route rank
    topk: int = 16             # top-k of every sparse propagation and transition
    s_window: int = 32         # window of the sequence propagations
    warmup: int = 2            # S warmup propagations
    blocks: int = 4            # joint blocks
    expanded: int = 256        # B_exp nodes
    compressed: int = 64       # B_cmp nodes
    refine: int = 2            # S refine propagations after the blocks
    query_refine: int = 2      # query transition + propagation rounds
    s_scale: float = 0.25      # merge scales of the paths
    b_scale: float = 0.20
    cross_scale: float = 0.15


def _merge(layer: Layer, delta: LayerDelta, scale: float, norm: nn.Module) -> Layer:
    """layer <- (tanh(state + a * delta_state), norm(val + a * delta_val))."""
    state = torch.tanh(layer.state + scale * delta.delta_state.to(layer.state.dtype))
    val = norm(layer.val + scale * delta.delta_val.to(layer.val.dtype))
    return layer.with_tensors(state=state, val=val)


def _slot_layer(template: Tensor, like: Layer) -> Layer:
    """A slot layer from a learned [nodes, 1 + dim] template (state, then value), per batch element of `like`."""
    t = template.to(like.val.dtype).expand(*like.state.shape[:-1], *template.shape)
    return Layer(dim=template.shape[1] - 1, num_nodes=template.shape[0], state=t[..., 0], val=t[..., 1:])


class _JointBlock(nn.Module):
    def __init__(self, cfg: ProgressiveBConfig, s_pairwise: nn.Module, implementation: str) -> None:
        super().__init__()
        d, r, k = cfg.dim, cfg.rank, cfg.topk

        def route() -> SparseTransition:
            return SparseTransition(LowRankBilinearRoute(d, d, rank=r), topk=k, implementation=implementation)

        def topk_prop() -> SparsePropagation:
            return SparsePropagation(LowRankBilinearPairwise(d, r), sparse_type="topk", topk=k,
                                     implementation=implementation)

        self.s_prop = SparsePropagation(s_pairwise, sparse_type="window", window=cfg.s_window,
                                        implementation=implementation)
        self.expand, self.exp_prop = route(), topk_prop()
        self.b_to_s, self.compress, self.s_to_b = route(), route(), route()
        self.cmp_prop = topk_prop()
        self.exp_slots = nn.Parameter(0.02 * torch.randn(cfg.expanded, d + 1))
        self.s_norm, self.exp_norm, self.cmp_norm = nn.LayerNorm(d), nn.LayerNorm(d), nn.LayerNorm(d)
        self.cfg = cfg

    def forward(self, s: Layer, cmp: Layer) -> tuple[Layer, Layer]:
        c = self.cfg
        s = _merge(s, self.s_prop.compute_delta(s), c.s_scale, self.s_norm)
        exp = _slot_layer(self.exp_slots, s)
        exp = _merge(exp, self.expand.compute_delta(cmp, exp), c.b_scale, self.exp_norm)
        exp = _merge(exp, self.exp_prop.compute_delta(exp), c.b_scale, self.exp_norm)
        s = _merge(s, self.b_to_s.compute_delta(exp, s), c.cross_scale, self.s_norm)
        cmp = _merge(cmp, self.compress.compute_delta(exp, cmp), c.b_scale, self.cmp_norm)
        cmp = _merge(cmp, self.s_to_b.compute_delta(s, cmp), c.cross_scale, self.cmp_norm)
        cmp = _merge(cmp, self.cmp_prop.compute_delta(cmp), c.b_scale, self.cmp_norm)
        return s, cmp


class ProgressiveBStep(nn.Module):
    """Query-block language model step: ``loss = step(prefix_ids, target_ids)``.

    prefix_ids [B, prefix], target_ids [B, query] (int64).  The query slots see
    the shifted targets (a start token, then targets[:-1]) as their inputs and
    predict the targets; the loss is the mean cross entropy over all slots."""

    def __init__(self, cfg: ProgressiveBConfig = ProgressiveBConfig(), *, implementation: str = "native") -> None:
        super().__init__()
        d, r, k = cfg.dim, cfg.rank, cfg.topk
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab, d)
        self.positions = nn.Parameter(0.02 * torch.randn(cfg.prefix + cfg.query, d))
        self.state_init = nn.Linear(d, 1)
        nn.init.zeros_(self.state_init.weight)
        nn.init.zeros_(self.state_init.bias)
        self.s_norm = nn.LayerNorm(d)
        s_pairwise = LowRankBilinearPairwise(d, r)  # shared by every sequence propagation
        self.warmup = nn.ModuleList(
            SparsePropagation(s_pairwise, sparse_type="window", window=cfg.s_window, implementation=implementation)
            for _ in range(cfg.warmup))
        self.blocks = nn.ModuleList(_JointBlock(cfg, s_pairwise, implementation) for _ in range(cfg.blocks))
        self.cmp_slots = nn.Parameter(0.02 * torch.randn(cfg.compressed, d + 1))  # B_cmp before the first block
        self.refine = nn.ModuleList(
            SparsePropagation(s_pairwise, sparse_type="window", window=cfg.s_window, implementation=implementation)
            for _ in range(cfg.refine))
        self.q_transition = SparseTransition(LowRankBilinearRoute(d, d, rank=r), topk=k, implementation=implementation)
        # a window of query - 1 over the query slots: causal dense propagation
        self.q_prop = SparsePropagation(LowRankBilinearPairwise(d, r), sparse_type="window", window=cfg.query - 1,
                                        implementation=implementation)
        self.q_norm = nn.LayerNorm(d)
        self.feedback_norm = nn.LayerNorm(d)
        self.feedback_proj = nn.Linear(d, d)
        self.head = nn.Sequential(nn.LayerNorm(d), nn.Linear(d, 4 * d), nn.GELU(), nn.Linear(4 * d, cfg.vocab))
        self.start_token = cfg.vocab - 1

    def _layer(self, val: Tensor, norm: nn.Module) -> Layer:
        state = torch.tanh(self.state_init(val).squeeze(-1))
        return Layer(dim=self.cfg.dim, num_nodes=val.shape[-2], state=state, val=norm(val))

    def encode_prefix(self, prefix_ids: Tensor) -> Layer:
        c = self.cfg
        s = self._layer(self.embed(prefix_ids) + self.positions[: prefix_ids.shape[-1]], self.s_norm)
        for op in self.warmup:
            s = _merge(s, op.compute_delta(s), c.s_scale, self.s_norm)
        cmp = _slot_layer(self.cmp_slots, s)
        for block in self.blocks:
            s, cmp = block(s, cmp)
        for op in self.refine:
            s = _merge(s, op.compute_delta(s), c.s_scale, self.s_norm)
        return s

    def query_logits(self, s: Layer, target_ids: Tensor) -> Tensor:
        c = self.cfg
        q_len = target_ids.shape[-1]
        shifted = torch.cat([torch.full_like(target_ids[:, :1], self.start_token), target_ids[:, :-1]], dim=1)
        feedback = self.feedback_proj(self.feedback_norm(self.embed(shifted)))
        start = s.num_nodes
        q = self._layer(feedback + self.positions[start:start + q_len], self.q_norm)
        for _ in range(c.query_refine):
            q = _merge(q, self.q_transition.compute_delta(s, q), c.cross_scale, self.q_norm)
            q = _merge(q, self.q_prop.compute_delta(q), c.s_scale, self.q_norm)
        return self.head(q.val)

    def forward(self, prefix_ids: Tensor, target_ids: Tensor) -> Tensor:
        logits = self.query_logits(self.encode_prefix(prefix_ids), target_ids)
        if logits.dtype in (torch.float16, torch.bfloat16):
            logits = logits.float()  # the loss of half-precision logits is taken in fp32
        return F.cross_entropy(logits.reshape(-1, logits.shape[-1]), target_ids.reshape(-1))
