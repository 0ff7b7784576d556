"""The Progressive-B query-block training step, composed from the hot-path operators.

This is the caller of the native path that BASELINE config 5 times, built as the
reference's ProgressiveBExampleLM builds it (scripts/progressive_b_example.py)
with every propagation and transition low-rank (route and pairwise rank r), so
that with implementation="native" each operator runs on the HIP library:

* a token prefix becomes a sequence layer S: token embedding plus a learned
  position encoding (an MLP of the node's position in [0, 1]), a linear state
  head, then the stabilisation every layer update ends with: state <- tanh(state),
  val <- LayerNorm(val) (initialize_sequence_layer, :1691-1719; _stabilize_layer,
  :282-292);
* S warmup windows (:1862-1870), whose deltas enter with the warmup scale (0 by
  default, so only the stabilisation changes S);
* joint blocks (ProgressiveBJointBlock.forward, :1108-1323) exchanging between S
  and two slot layers, an expanded layer B_exp (fresh from learned templates in
  every block) and a compressed layer B_cmp (from templates in the first block,
  then carried): S window; B_cmp -> B_exp transition and B_exp top-k; B_exp -> S;
  B_exp -> B_cmp, S -> B_cmp and B_cmp top-k.  Each update replaces the layer by
  the scaled delta (block_residual off: _scaled_apply, :1011-1024) with the
  stage's path scales (alpha_b, beta_s_to_b, beta_b_to_s: the lite and mid
  stages of build_progressive_b_stage_specs, :713-781), then stabilises;
* S refine windows at scale 0.25 (:1895-1898);
* the teacher-forced query block (forward_query_block, :2059-2152): query slots
  take the feedback of the shifted targets (start token, then targets[:-1]) --
  embedding, LayerNorm, linear -- as their values, the state head as their
  state, and run `query_refine` rounds of transition S -> Q (:1957-1975) and
  causal propagation over Q (a window of Q - 1, :1977-2012); the head is
  LayerNorm, Linear(d, 4d), GELU, Linear(4d, vocab); the loss is the mean cross
  entropy (compute_next_token_loss with front weight 1, :2997-3006).

Options this step does not take (dropouts, route-concentration and diversity
losses, stats tracking, the pre-norm position, residual merges) are the
reference's off-by-default ones.  The compressed adapter (a dense bilinear
transition used when B_cmp changes size between stages, :1078-1087) is not
built: every block here keeps one B_cmp size.  The first slot positions of the
query layer (initialize_query_layer, :1918-1939) are replaced by the feedback
before use, so they are not computed.
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

# (alpha_b, beta_s_to_b, beta_b_to_s) of the reference's lite and mid stages
# (build_progressive_b_stage_specs defaults, scripts/progressive_b_example.py:719-726)
LITE_STAGE = (0.3, 0.25, 0.15)
MID_STAGE = (0.65, 0.55, 0.35)


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
    blocks: int = 4            # joint blocks: the first half lite, the rest mid
    expanded: int = 256        # B_exp nodes
    compressed: int = 64       # B_cmp nodes
    refine: int = 2            # S refine propagations after the blocks
    query_refine: int = 2      # query transition + propagation rounds
    s_scale: float = 0.25      # s_delta_scale
    b_scale: float = 0.20      # b_delta_scale
    cross_scale: float = 0.15  # cross_delta_scale
    warmup_scale: float = 0.0  # warmup_delta_scale
    refine_scale: float = 0.25

    def stage(self, block: int) -> tuple[float, float, float]:
        """(alpha_b, beta_s_to_b, beta_b_to_s) of a joint block."""
        return LITE_STAGE if block < (self.blocks + 1) // 2 else MID_STAGE


def _replace_scaled(layer: Layer, delta: LayerDelta, scale: float) -> Layer:
    """The layer replaced by the scaled delta (merge "replace"); a zero scale keeps it."""
    if scale == 0.0:
        return layer
    return layer.with_tensors(state=delta.delta_state * scale, val=delta.delta_val * scale)


def _stabilize(layer: Layer, norm: nn.Module) -> Layer:
    return layer.with_tensors(state=torch.tanh(layer.state), val=norm(layer.val))


class PositionEncoding(nn.Module):
    """An MLP (Linear(1, w), SiLU, Linear(w, dim), w = max(dim, 8)) of each node's
    position on [0, 1] (reference modules.py:706-739, LearnedPositionEncoding)."""

    def __init__(self, dim: int) -> None:
        super().__init__()
        width = max(dim, 8)
        self.net = nn.Sequential(nn.Linear(1, width), nn.SiLU(), nn.Linear(width, dim))

    def forward(self, num_nodes: int, *, device=None, dtype=None) -> Tensor:
        w = self.net[0].weight
        if num_nodes == 1:
            pos = torch.zeros(1, 1, device=device, dtype=w.dtype)
        else:
            pos = torch.linspace(0.0, 1.0, num_nodes, device=device, dtype=w.dtype).unsqueeze(-1)
        out = self.net(pos)
        return out if dtype is None else out.to(dtype)


def _slot_layer(state_t: Tensor, val_t: Tensor, like: Layer) -> Layer:
    """A slot layer from learned templates, one copy per batch element of `like`."""
    batch = tuple(like.state.shape[:-1])
    state = state_t.expand(*batch, *state_t.shape).to(device=like.state.device, dtype=like.state.dtype)
    val = val_t.expand(*batch, *val_t.shape).to(device=like.val.device, dtype=like.val.dtype)
    return Layer(dim=val_t.shape[-1], num_nodes=state_t.shape[0], state=state, val=val)


class _JointBlock(nn.Module):
    """One ProgressiveBJointBlock (reference :786-1323) with low-rank operators;
    the sequence, expanded and compressed pairwise modules are shared by all blocks."""

    def __init__(self, cfg: ProgressiveBConfig, stage: tuple[float, float, float], s_pairwise: nn.Module,
                 exp_pairwise: nn.Module, cmp_pairwise: nn.Module, implementation: str) -> None:
        super().__init__()
        d, r, k = cfg.dim, cfg.rank, cfg.topk
        self.cfg = cfg
        self.alpha_b, self.beta_s_to_b, self.beta_b_to_s = stage
        self.s_norm, self.exp_norm, self.cmp_norm = nn.LayerNorm(d), nn.LayerNorm(d), nn.LayerNorm(d)
        self.exp_slot_state = nn.Parameter(0.02 * torch.randn(cfg.expanded))
        self.exp_slot_val = nn.Parameter(0.02 * torch.randn(cfg.expanded, d))
        self.cmp_slot_state = nn.Parameter(0.02 * torch.randn(cfg.compressed))
        self.cmp_slot_val = nn.Parameter(0.02 * torch.randn(cfg.compressed, d))

        def route() -> SparseTransition:
            return SparseTransition(LowRankBilinearRoute(d, d, rank=r), topk=k, implementation=implementation)

        self.s_prop = SparsePropagation(s_pairwise, sparse_type="window", window=cfg.s_window,
                                        implementation=implementation)
        self.expand = route()
        self.exp_prop = SparsePropagation(exp_pairwise, sparse_type="topk", topk=min(k, cfg.expanded),
                                          implementation=implementation)
        self.b_to_s = route()
        self.compress = route()
        self.s_to_b = route()
        self.cmp_prop = SparsePropagation(cmp_pairwise, sparse_type="topk", topk=min(k, cfg.compressed),
                                          implementation=implementation)

    def forward(self, s: Layer, cmp: Layer | None) -> tuple[Layer, Layer]:
        c = self.cfg
        a = self.alpha_b
        s = _stabilize(_replace_scaled(s, self.s_prop.compute_delta(s), c.s_scale), self.s_norm)
        if cmp is None:
            cmp = _slot_layer(self.cmp_slot_state, self.cmp_slot_val, s)
        elif cmp.num_nodes != c.compressed:
            raise NotImplementedError("B_cmp changes size between blocks: the compressed adapter is not built")
        cmp = _stabilize(cmp, self.cmp_norm)

        exp = _slot_layer(self.exp_slot_state, self.exp_slot_val, s)
        exp = _replace_scaled(exp, self.expand.compute_delta(cmp, exp), a * c.b_scale)
        exp = _replace_scaled(exp, self.exp_prop.compute_delta(exp), a * c.b_scale)
        exp = _stabilize(exp, self.exp_norm)

        s = _replace_scaled(s, self.b_to_s.compute_delta(exp, s), a * self.beta_b_to_s * c.cross_scale)
        s = _stabilize(s, self.s_norm)

        nxt = _replace_scaled(cmp, self.compress.compute_delta(exp, cmp), a * c.b_scale)
        nxt = _replace_scaled(nxt, self.s_to_b.compute_delta(s, nxt), a * self.beta_s_to_b * c.cross_scale)
        nxt = _replace_scaled(nxt, self.cmp_prop.compute_delta(nxt), a * c.b_scale)
        return s, _stabilize(nxt, self.cmp_norm)


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
        self.positions = PositionEncoding(d)
        self.state_init = nn.Linear(d, 1)
        nn.init.zeros_(self.state_init.weight)
        nn.init.zeros_(self.state_init.bias)
        self.s_norm = nn.LayerNorm(d)
        # one pairwise module per layer family, shared by every operator of the family
        s_pairwise, exp_pairwise = LowRankBilinearPairwise(d, r), LowRankBilinearPairwise(d, r)
        cmp_pairwise, q_pairwise = LowRankBilinearPairwise(d, r), LowRankBilinearPairwise(d, r)
        self.q_norm = nn.LayerNorm(d)
        self.q_transition = SparseTransition(LowRankBilinearRoute(d, d, rank=r), topk=k, implementation=implementation)
        # the query propagation runs as a causal window of query - 1 over the slots
        self.q_prop = SparsePropagation(q_pairwise, sparse_type="window", window=cfg.query - 1,
                                        implementation=implementation)
        self.warmup = nn.ModuleList(
            SparsePropagation(s_pairwise, sparse_type="window", window=cfg.s_window, implementation=implementation)
            for _ in range(cfg.warmup))
        self.blocks = nn.ModuleList(
            _JointBlock(cfg, cfg.stage(i), s_pairwise, exp_pairwise, cmp_pairwise, implementation)
            for i in range(cfg.blocks))
        self.refine = nn.ModuleList(
            SparsePropagation(s_pairwise, sparse_type="window", window=cfg.s_window, implementation=implementation)
            for _ in range(cfg.refine))
        self.head_norm = nn.LayerNorm(d)
        self.feedback_norm = nn.LayerNorm(d)
        self.feedback_proj = nn.Linear(d, d)
        self.head = nn.Sequential(nn.Linear(d, 4 * d), nn.GELU(), nn.Linear(4 * d, cfg.vocab))
        self.start_token = cfg.vocab - 1

    def encode_prefix(self, prefix_ids: Tensor) -> Layer:
        c = self.cfg
        val = self.embed(prefix_ids)
        val = val + self.positions(prefix_ids.shape[-1], device=val.device, dtype=val.dtype).unsqueeze(0)
        s = Layer(dim=c.dim, num_nodes=val.shape[-2], state=self.state_init(val).squeeze(-1), val=val)
        s = _stabilize(s, self.s_norm)
        for op in self.warmup:
            s = _stabilize(_replace_scaled(s, op.compute_delta(s), c.warmup_scale), self.s_norm)
        cmp = None
        for block in self.blocks:
            s, cmp = block(s, cmp)
        for op in self.refine:
            s = _stabilize(_replace_scaled(s, op.compute_delta(s), c.refine_scale), self.s_norm)
        return s

    def query_logits(self, s: Layer, target_ids: Tensor) -> Tensor:
        c = self.cfg
        shifted = torch.cat([torch.full_like(target_ids[:, :1], self.start_token), target_ids[:, :-1]], dim=1)
        feedback = self.feedback_proj(self.feedback_norm(self.embed(shifted)))
        q = Layer(dim=c.dim, num_nodes=shifted.shape[-1], state=self.state_init(feedback).squeeze(-1), val=feedback)
        q = _stabilize(q, self.q_norm)
        for _ in range(c.query_refine):
            q = _stabilize(_replace_scaled(q, self.q_transition.compute_delta(s, q), c.cross_scale), self.q_norm)
            q = _stabilize(_replace_scaled(q, self.q_prop.compute_delta(q), c.s_scale), self.q_norm)
        return self.head(self.head_norm(q.val))

    def forward(self, prefix_ids: Tensor, target_ids: Tensor) -> Tensor:
        logits = self.query_logits(self.encode_prefix(prefix_ids), target_ids)
        if logits.dtype in (torch.float16, torch.bfloat16):
            logits = logits.float()  # the loss of half-precision logits is taken in fp32
        return F.cross_entropy(logits.reshape(-1, logits.shape[-1]), target_ids.reshape(-1))
