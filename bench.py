"""Benchmark of the native hot path on one MI355X.

Default workload (top-k variant, the headline metric):
SparsePropagation top-k with LowRankBilinearPairwise, B=16, N=4096, D=512,
r=64, k=32, fp32, val rows unit-norm, state ~ N(0,1), default module init; one
step = forward + backward of loss = sum(delta_state) + sum(delta_val) through
the jakal_net API with implementation="native".

Other workloads (--workload), one per hot-path row, same output format:
  c2-window   BASELINE config 2: window propagation, B=8, T=1024, D=384, r=32,
              window 64, val and state ~ N(0,1), default init.
  c3-transition BASELINE config 3: SparseTransition S->B (1024 -> 256 nodes) then
              B->S (256 -> 1024), B=8, D=512, r=64, top-16 per source, softmax
              routes, states and vals ~ N(0,1), default init.
  c4-dense    BASELINE config 4, dense variant: Propagation over all N x N pairs,
              B=16, N=4096, D=512, r=64, softsign, inputs as c4-topk.
  c4-topk-bf16 BASELINE config 4 (C4-topk bf16 row): c4-topk with bf16 layer
              states and values; the value rows move as bf16 and the top-k
              scores run on bf16 MFMAs (sparse-byte budget 6.72 GB).
  c4-dense-bf16 c4-dense with bf16 layer states and values: the N x N
              products on bf16 MFMA.
  c4-dense-causal c4-dense with a full causal window (the masked half skipped).
  c3-transition-dense C3 sizes with every source routed to every destination.
  c5-progressive-b BASELINE config 5: the Progressive-B query-block training
              step (forward, backward, AdamW; tokens/s).

Inputs and parameters are resident in HBM before the timed region.

Timing.  The step is first run `steps` times eagerly with the library's
per-kernel HIP events on the launch stream (the kernel table and roofline).
Then it is captured once into a HIP graph
(torch.cuda.CUDAGraph; the library only launches kernels, so the whole
forward+backward captures) and `steps` back-to-back replays are timed:
`value` and `ms_per_step` come from the replays, the eager figures are
reported under `graph`.  --eager times the eager steps only.  C5's step
(forward, backward, AdamW) captures as a whole with AdamW's capturable state
and an autocast without cast cache.

Prints one JSON line:
  value        routed pairs per second (edges aggregated per step / step time)
  roofline     dominant kernel: algorithmic bytes (or flops) per launch / its
               average duration, measured with HIP events over the eager timed
               region; `traffic` = HBM-side bytes per launch measured by
               rocprofv3 FETCH_SIZE/WRITE_SIZE passes of this command
  kernels      the same figures for every kernel of the step; avg_ms_alone (and the
               HBM kernels' frac_alone) from a few more eager steps with the library's
               side streams off, so that no kernel shares the GPU with another
  hbm_measured_GBps, hbm_frac
               step-level HBM-side traffic: the rocprofv3 FETCH_SIZE + WRITE_SIZE bytes
               per launch of every kernel (profiles/<workload>_hbm_traffic.json) times
               its launches per step, over ms_per_step, and its fraction of 8 TB/s
               (details under `hbm`, with the compulsory bytes of the HBM-bound kernels)
  sparse_phase_algorithmic_GBps
               BASELINE's sparse-phase bytes (no cache reuse) over ms_per_step: an
               algorithmic rate; above 8 TB/s it says the step is not HBM-bound
  cpu_baseline the same workload through the operator API's implementation="reference"
               backend on the host cores (warmup 1, median of 3)

The top-k select's flops are fp32-equivalent score products (2 r per pair),
priced against the fp32 MFMA peak.  With --select-mode split-f16 (the
library default) the MFMA pipe runs three fp16 products for each (hi.hi +
hi.lo + lo.hi of two-term fp16 operand splits, fp32 accumulation); that
kernel entry also reports the executed fp16 MFMA rate against its own peak.

  python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--workload c4-topk] [--no-cpu-baseline]
                  [--select-mode split-f16|f32] [--gemm-tile 0|64|128] [--eager]
  python bench.py --calibrate-copy     # plain 1 GiB device copy (counter scale)
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "jakal-net_amd"))

HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
FP16_MFMA_PEAK_TFLOPS = 2500.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
# gemm_x3_kernel computes each fp32 product as six bf16 MFMA products: its
# MFMA bound in fp32-equivalent flops
X3_PRODUCTS = 6
X3_MFMA_PEAK_TFLOPS = BF16_MFMA_PEAK_TFLOPS / X3_PRODUCTS
# split-fp16 select: fp16 MFMA products per fp32-equivalent product (hi.hi + hi.lo + lo.hi)
SPLIT_PRODUCTS = 3

# the headline workload (kept as module constants: the profile summaries use them)
CONFIG = {"batch": 16, "nodes": 4096, "dim": 512, "rank": 64, "topk": 32}


def rows_backward_split(nk: int, D: int, vb: int = 4) -> bool:
    """Whether the library runs the row backward's dot products as two column
    slabs first (rows_backward_dots_kernel): value rows of a batch element above
    2 MiB with 256 < D <= 1024 (jn_edges.hip, rows_backward_slab); vb bytes per
    value element."""
    return 256 < D <= 1024 and nk * D * vb > (2 << 20)


def fused_column_slabs(D: int, vb: int = 4) -> int:
    """Column slabs of the fused column pass of a top-k backward
    (cols_gather_dots_kernel: 64 lanes x 16 bytes per slab), 0 when it does not
    apply (rows not whole 16-byte packs, or more than two slabs;
    jn_edges.hip, cols_gather_dots_slabs)."""
    if (D * vb) % 16:
        return 0
    slabs = -(-D * vb // 1024)
    return slabs if slabs <= 2 else 0


def csr_table_bytes(M: int, Mk: int, B: int) -> float:
    """Bytes of the edge grouping's per-tile key counts for M query rows and Mk
    keys over B batch elements: tiles of whole 64-row chunks, about 256 over
    the batch, at most 1024 rows (jn_edges.hip, csr_tile_rows)."""
    nq, nk = M // B, Mk // B
    want = (M + 255) // 256
    rows = min(1024, max(64, -(-want // 64) * 64))
    return 4.0 * B * (-(-nq // rows)) * nk


def edge_kernel_model(name: str, M: int, E: int, D: int, r: int, split: bool | str = False,
                      Mk: int | None = None, vb: float = 4.0, batch: int = 1) -> tuple | None:
    """(bound, algorithmic bytes or flops, compulsory bytes) of the edge-list kernels.

    M = aggregated (query) rows, Mk = source (key) rows (M for propagation),
    E = routed pairs.  Algorithmic bytes count every operand once per use (an
    edge gathers one D-row of fp32 values, its index and score), so they
    credit no cache reuse; compulsory bytes count each distinct input row once
    and each output once: the HBM bytes no schedule can avoid.  The gathers
    reuse each value row about k times from L2, so their algorithmic rate is an
    L2-side figure and their HBM roofline fraction is priced on compulsory bytes.
    split: the row backward runs as dots + finish ("fused": its dots come from
    the fused column pass, read through the record indices).  vb: bytes per value-row
    element (4 fp32, 2 bf16); projections, scores and edge records stay fp32.
    batch: batch elements of the edge list (the edge grouping's tiling)."""
    Mk = M if Mk is None else Mk
    D4 = vb * D  # bytes of one value row
    if name.startswith("rows_forward_kernel"):
        # idx+score+ps per edge, pv row per edge; delta_val row + delta_state per row
        return ("hbm", E * (12.0 + D4) + M * (D4 + 4.0),
                E * 8.0 + Mk * (D4 + 4.0) + M * (D4 + 4.0))
    if name.startswith("rows_backward_dots_kernel"):
        # idx, pv row, partial-dot write per edge; grad-delta row per row
        return ("hbm", E * (4.0 + D4 + 4.0) + M * D4,
                E * 12.0 + (M + Mk) * D4)
    if name.startswith("cols_gather_dots_kernel"):
        # per edge and slab: record, grad-delta row slab, gds[row], partial-dot write;
        # per column: segment bounds, pv row, grad_pv row, grad_ps
        slabs = max(1, fused_column_slabs(D, int(vb)))
        return ("hbm", E * (slabs * 24.0 + D4) + Mk * (8.0 + 2.0 * D4 + 4.0),
                E * (16.0 + 4.0 * slabs) + M * (D4 + 4.0) + Mk * (2.0 * D4 + 8.0))
    if name.startswith("csr_count_kernel"):
        # edge index per edge; per-tile counts of every key
        table = csr_table_bytes(M, Mk, batch)
        return ("hbm", E * 4.0 + table, E * 4.0 + table)
    if name.startswith("csr_tile_prefix_kernel"):
        # the per-tile counts read and rewritten, the degree row written
        table = csr_table_bytes(M, Mk, batch)
        return ("hbm", 2.0 * table + Mk * 4.0, 2.0 * table + Mk * 4.0)
    if name.startswith("csr_fill_kernel"):
        # edge index, score, record and record index per edge; each tile's row
        # of the table and the batch element's degree row (read by every tile)
        table = csr_table_bytes(M, Mk, batch)
        tiles = table / (4.0 * Mk)
        return ("hbm", E * (4.0 + 4.0 + 16.0 + 4.0) + table + tiles * Mk * 4.0,
                E * (4.0 + 4.0 + 16.0 + 4.0) + table + Mk * 4.0)
    if name.startswith("rows_backward_kernel"):
        if split == "fused":
            # idx+score, record index, two partial dots, ps, key row, gsc write per edge;
            # grad-delta state, dq row, row sum per row
            return ("hbm", E * (8.0 + 4.0 + 8.0 + 4.0 + 4.0 * r + 4.0) + M * (4.0 + 4.0 * r + 4.0),
                    E * 28.0 + Mk * (4.0 + 4.0 * r) + M * (8.0 + 4.0 * r))
        if split:
            # idx+score, two partial dots, ps, key row, gsc+coef writes per edge;
            # grad-delta state, dq row, row sum per row
            return ("hbm", E * (8.0 + 8.0 + 4.0 + 4.0 * r + 8.0) + M * (4.0 + 4.0 * r + 4.0),
                    E * 24.0 + Mk * (4.0 + 4.0 * r) + M * (8.0 + 4.0 * r))
        # idx+score, ps, pv row, key row per edge; gsc+coef writes per edge;
        # grad-delta row + state, dq row, row sum per row
        return ("hbm", E * (8.0 + 4.0 + D4 + 4.0 * r + 8.0) + M * (D4 + 4.0 + 4.0 * r + 4.0),
                E * 16.0 + Mk * (D4 + 4.0 * r + 4.0) + M * (D4 + 4.0 * r + 8.0))
    if name.startswith("cols_gather_kernel"):
        # edge record, grad-delta row per edge; segment bounds, grad_pv row, grad_ps per column
        return ("hbm", E * (16.0 + D4) + Mk * (8.0 + D4 + 4.0),
                E * 16.0 + M * D4 + Mk * (D4 + 8.0))
    if name.startswith("cols_keygrad_kernel"):
        # edge record, query row per edge; segment bounds, dk row, key row per column
        return ("hbm", E * (16.0 + 4.0 * r) + Mk * (8.0 + 8.0 * r),
                E * 16.0 + M * 4.0 * r + Mk * (8.0 * r + 4.0))
    if name.startswith("window_scores_kernel"):
        # query row per row; key row per edge; idx + score written per edge
        return ("hbm", E * (4.0 * r + 8.0) + M * 4.0 * r, E * 8.0 + (M + Mk) * 4.0 * r)
    if name.startswith("gemm_f32_kernel"):
        return ("mfma", 2.0 * M * D * 2 * r, None)
    if name.startswith("gemm_bf16_kernel"):
        # bf16 layers: projections and their gradients on bf16 MFMA
        return ("mfma", 2.0 * M * D * 2 * r, None, BF16_MFMA_PEAK_TFLOPS)
    return None


def split_prep_model(name: str, key_rows: float, r: int) -> tuple | None:
    """The split-fp16 select's two prep kernels over key_rows key rows per launch:
    a max-|key| pass (reads the keys) and the split (reads them again, writes
    hi and lo fp16 planes of the rank rounded up to 32)."""
    rp = -(-r // 32) * 32
    if name.startswith("select_split_absmax_kernel"):
        return "hbm", key_rows * 4.0 * r, key_rows * 4.0 * r
    if name.startswith("select_split_keys_kernel"):
        return "hbm", key_rows * (4.0 * r + 4.0 * rp), key_rows * (4.0 * r + 4.0 * rp)
    return None


def kernel_model(name: str, B: int, N: int, D: int, r: int, k: int, bf16: bool = False) -> tuple | None:
    """Kernel model of the top-k workload (bf16: bf16 value rows and bf16 select
    operands, priced against the bf16 MFMA peak)."""
    if name.startswith("lowrank_topk_select_kernel"):
        return "mfma", 2.0 * B * N * N * r, None, BF16_MFMA_PEAK_TFLOPS if bf16 else FP32_MFMA_PEAK_TFLOPS
    if name.startswith("select_split_"):
        return split_prep_model(name, B * N, r)
    if name.startswith("select_bf16_keys_kernel"):
        # reads the fp32 key rows, writes bf16 rows of the rank rounded up to 32
        rp = -(-r // 32) * 32
        return "hbm", B * N * (4.0 * r + 2.0 * rp), B * N * (4.0 * r + 2.0 * rp)
    vb = 2 if bf16 else 4
    split = "fused" if fused_column_slabs(D, vb) else rows_backward_split(N, D, vb)
    return edge_kernel_model(name, B * N, B * N * k, D, r, split, vb=float(vb), batch=B)


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(wl, torch) -> dict:
    """The same workload through the operator API's implementation="reference"
    backend (the dense masked PyTorch form of propagation.py:453-480 /
    transition.py:431-452) on the host cores: torch threads = the host's
    cores (capped by OMP_NUM_THREADS when set, the CPU share a GPU box grants),
    one warmup, the median of three timed forward+backward steps of loss =
    sum(delta_state) + sum(delta_val).  The sample is the whole workload, or
    `cpu_batch` of its batch elements where the dense [B, N, N] reference form
    would take tens of seconds per step; pairs/s is scaled to the sample."""
    cores = os.cpu_count() or 1
    share = os.environ.get("OMP_NUM_THREADS")
    threads = min(cores, int(share)) if share and share.isdigit() and int(share) > 0 else cores
    full = wl.config["batch"]
    batch = min(full, getattr(wl, "cpu_batch", full))
    saved = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        step = workload_step(wl, torch, torch.device("cpu"), impl="reference", batch=batch)
        step()
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            step()
            times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(saved)
    t = sorted(times)[1]
    what = "the whole workload" if batch == full else f"{batch} of its {full} batch elements"
    return {
        "value": wl.edges() * batch / full / t,
        "unit": getattr(wl, "unit", "routed pairs/s"),
        "cores": threads,
        "kind": "port",
        "sample": f"{what} ({wl.workload.replace(', native', '')}) through implementation='reference' on "
                  f"the CPU, fp32, torch threads {threads} (os.cpu_count() {cores}), warmup 1, median of 3: "
                  f"{t:.3f} s per step",
        "cpu_model": _cpu_model(),
        "os_cpu_count": cores,
        "torch_threads": threads,
        "step_s": [round(x, 4) for x in times],
    }


def _make_step(torch, op, layer):
    """One forward+backward of loss = sum of every delta tensor (grads cleared first)."""
    if layer is None:  # a multi-module step: op supplies its own loss terms
        ones = [torch.ones_like(t) for t in op.loss_terms()]

        def step() -> None:
            op.zero_grad(set_to_none=True)
            torch.autograd.backward(op.loss_terms(), ones)
        return step

    ones_s = torch.ones_like(layer.state)
    ones_v = torch.ones_like(layer.val)

    def step() -> None:
        op.zero_grad(set_to_none=True)
        layer.val.grad = None
        layer.state.grad = None
        delta = op(layer)
        torch.autograd.backward([delta.delta_state, delta.delta_val], [ones_s, ones_v])
    return step


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------
class TopkC4:
    name = "c4-topk"
    metric = "routed pairs/sec + HBM GB/s (% peak), SparsePropagation N=4096 D=512 k=32 fwd+bwd"
    workload = "C4-topk SparsePropagation fwd+bwd, LowRankBilinearPairwise, native"
    data = "synthetic (seeded N(0,1) state, unit-norm N(0,1) val rows, default module init)"
    config = CONFIG
    traffic_file = "c4_topk_hbm_traffic.json"
    cpu_batch = 2  # CPU baseline sample: 2 of the 16 batch elements (about 3 s per step on 16 cores)

    def edges(self) -> int:
        c = self.config
        return c["batch"] * c["nodes"] * c["topk"]

    def model(self, name):
        c = self.config
        return kernel_model(name, c["batch"], c["nodes"], c["dim"], c["rank"], c["topk"])

    def sparse_bytes(self) -> float:
        # hot-path algorithmic bytes per fwd+bwd (gathers, scatters, edge records, state)
        c = self.config
        E, M, D = self.edges(), c["batch"] * c["nodes"], c["dim"]
        return 3 * 4 * D * (E + M) + 24 * E + 3 * 4 * (E + M)

    def build(self, torch, dev, impl: str = "native", batch: int | None = None):
        from jakal_net import Layer, LowRankBilinearPairwise, SparsePropagation

        B, N, D, r, k = (self.config[x] for x in ("batch", "nodes", "dim", "rank", "topk"))
        B = batch or B
        g = torch.Generator().manual_seed(1004)
        state = torch.randn(B, N, generator=g)
        val = torch.randn(B, N, D, generator=g)
        val = val / val.norm(dim=-1, keepdim=True)
        torch.manual_seed(1004)
        op = SparsePropagation(LowRankBilinearPairwise(D, r), sparse_type="topk", topk=k,
                               implementation=impl).to(dev)
        return op, Layer(dim=D, num_nodes=N, state=state.to(dev).requires_grad_(True),
                         val=val.to(dev).requires_grad_(True))


class TopkC4Bf16(TopkC4):
    """c4-topk with bf16 layer states and values (BASELINE C4-topk bf16 row)."""

    name = "c4-topk-bf16"
    metric = ("routed pairs/sec + HBM GB/s (% peak), SparsePropagation N=4096 D=512 k=32 fwd+bwd, "
              "bf16 activations")
    workload = "C4-topk bf16 SparsePropagation fwd+bwd, LowRankBilinearPairwise, bf16 layers, native"
    data = ("synthetic (seeded N(0,1) state, unit-norm N(0,1) val rows, both rounded to bf16; default module "
            "init, fp32 weights)")
    dtype = "bf16"
    traffic_file = "c4_topk_bf16_hbm_traffic.json"
    cpu_batch = 1

    def model(self, name):
        c = self.config
        return kernel_model(name, c["batch"], c["nodes"], c["dim"], c["rank"], c["topk"], bf16=True)

    def sparse_bytes(self) -> float:
        # TopkC4's budget with 2-byte value rows (6.72 GB per step)
        c = self.config
        E, M, D = self.edges(), c["batch"] * c["nodes"], c["dim"]
        return 3 * 2 * D * (E + M) + 24 * E + 3 * 4 * (E + M)

    def build(self, torch, dev, impl: str = "native", batch: int | None = None):
        from jakal_net import Layer

        op, layer = super().build(torch, dev, impl=impl, batch=batch)
        bf = lambda t: t.detach().bfloat16().requires_grad_(True)  # noqa: E731
        return op, Layer(dim=layer.dim, num_nodes=layer.num_nodes, state=bf(layer.state), val=bf(layer.val))


class WindowC2:
    name = "c2-window"
    metric = "routed pairs/sec + HBM GB/s (% peak), SparsePropagation window T=1024 D=384 w=64 fwd+bwd"
    workload = "C2-window SparsePropagation fwd+bwd, LowRankBilinearPairwise, native"
    data = "synthetic (seeded N(0,1) state and val, default module init)"
    config = {"batch": 8, "nodes": 1024, "dim": 384, "rank": 32, "window": 64}
    traffic_file = "c2_window_hbm_traffic.json"

    def edges(self) -> int:
        c = self.config
        width = min(c["window"] + 1, c["nodes"])
        return c["batch"] * sum(min(i + 1, width) for i in range(c["nodes"]))

    def model(self, name):
        c = self.config
        return edge_kernel_model(name, c["batch"] * c["nodes"], self.edges(), c["dim"], c["rank"],
                                 rows_backward_split(c["nodes"], c["dim"]))

    def sparse_bytes(self) -> float:
        # contiguous bands: compulsory dense bytes (read val, write delta; bwd read grad, read val, write grad)
        c = self.config
        return 5 * 4 * c["batch"] * c["nodes"] * c["dim"]

    def build(self, torch, dev, impl: str = "native", batch: int | None = None):
        from jakal_net import Layer, LowRankBilinearPairwise, SparsePropagation

        B, N, D, r, w = (self.config[x] for x in ("batch", "nodes", "dim", "rank", "window"))
        B = batch or B
        g = torch.Generator().manual_seed(1002)
        state = torch.randn(B, N, generator=g)
        val = torch.randn(B, N, D, generator=g)
        torch.manual_seed(1002)
        op = SparsePropagation(LowRankBilinearPairwise(D, r), sparse_type="window", window=w,
                               implementation=impl).to(dev)
        return op, Layer(dim=D, num_nodes=N, state=state.to(dev).requires_grad_(True),
                         val=val.to(dev).requires_grad_(True))


class TransitionC3:
    name = "c3-transition"
    metric = "routed pairs/sec + HBM GB/s (% peak), SparseTransition S->B and B->S N_src=1024 N_dst=256 D=512 k=16 fwd+bwd"
    workload = "C3 SparseTransition S->B then B->S fwd+bwd, LowRankBilinearRoute, softmax routes, native"
    data = "synthetic (seeded N(0,1) states and vals, default module init)"
    config = {"batch": 8, "s_nodes": 1024, "b_nodes": 256, "dim": 512, "rank": 64, "topk": 16}
    traffic_file = "c3_transition_hbm_traffic.json"

    def edges(self) -> int:
        c = self.config
        return c["batch"] * (c["s_nodes"] + c["b_nodes"]) * c["topk"]

    def model(self, name):
        c = self.config
        B, S, Bn, D, r, k = (c[x] for x in ("batch", "s_nodes", "b_nodes", "dim", "rank", "topk"))
        E, rows = self.edges(), B * (S + Bn)
        if name.startswith("lowrank_topk_select_kernel") or name.startswith("select_small_kernel"):
            return "mfma", 2.0 * B * S * Bn * r  # per launch: one direction scores its S x B pairs
        if name.startswith("select_split_"):
            return split_prep_model(name, B * (S + Bn) / 2, r)  # keys: B rows one way, S rows the other
        # per launch = half of both directions; `rows` counts source rows of both
        # directions, which are also the destination rows of both
        if name.startswith("route_rows_backward_kernel"):
            # per edge: idx + logit + grad-delta row of the destination + its key row + g_logit write;
            # per source row: its value row, its grad-value write, dq write.  Compulsory: each
            # destination's grad-delta and key rows once
            return ("hbm", (E * (8.0 + 4.0 * D + 4.0 * r + 4.0) + rows * (8.0 * D + 4.0 * r + 16.0)) / 2,
                    (E * 12.0 + rows * (8.0 * D + 4.0 * r + 16.0) + rows * (4.0 * D + 4.0 * r)) / 2)
        if name.startswith("route_gather_kernel") or name.startswith("cols_gather_kernel"):
            # per edge: edge record + source value row; per destination: delta row write
            return ("hbm", (E * (16.0 + 4.0 * D) + rows * (4.0 * D + 12.0)) / 2,
                    (E * 16.0 + rows * (8.0 * D + 12.0)) / 2)
        if name.startswith("cols_keygrad_kernel"):
            # per edge: edge record + source projection row; per destination: dk row + its projection row
            return ("hbm", (E * (16.0 + 4.0 * r) + rows * (8.0 + 8.0 * r)) / 2,
                    (E * 16.0 + rows * (12.0 * r + 4.0)) / 2)
        if name.startswith("gemm_f32_kernel"):
            return "mfma", 2.0 * rows * D * r / 2
        return None

    def sparse_bytes(self) -> float:
        # SURVEY-style per direction: fwd scatter + bwd gather of dst rows (8DE), src val read twice +
        # grad written (3*4*D*M_src), dst rows (8*D*M_dst), edge records (24E); summed over both directions
        c = self.config
        B, S, Bn, D, k = (c[x] for x in ("batch", "s_nodes", "b_nodes", "dim", "topk"))
        tot = 0.0
        for ns, nd in ((S, Bn), (Bn, S)):
            E = B * ns * k
            tot += 8 * D * E + 3 * 4 * D * B * ns + 8 * D * B * nd + 24 * E
        return tot

    def build(self, torch, dev, impl: str = "native", batch: int | None = None):
        from jakal_net import Layer, LowRankBilinearRoute, SparseTransition

        c = self.config
        B, S, Bn, D, r, k = (c[x] for x in ("batch", "s_nodes", "b_nodes", "dim", "rank", "topk"))
        B = batch or B
        g = torch.Generator().manual_seed(1003)
        s_state, s_val = torch.randn(B, S, generator=g), torch.randn(B, S, D, generator=g)
        b_state, b_val = torch.randn(B, Bn, generator=g), torch.randn(B, Bn, D, generator=g)
        torch.manual_seed(1003)
        s_to_b = SparseTransition(LowRankBilinearRoute(D, D, rank=r), topk=k, implementation=impl).to(dev)
        b_to_s = SparseTransition(LowRankBilinearRoute(D, D, rank=r), topk=k, implementation=impl).to(dev)
        s_layer = Layer(dim=D, num_nodes=S, state=s_state.to(dev).requires_grad_(True),
                        val=s_val.to(dev).requires_grad_(True))
        b_layer = Layer(dim=D, num_nodes=Bn, state=b_state.to(dev).requires_grad_(True),
                        val=b_val.to(dev).requires_grad_(True))
        return _TwoWayTransition(torch, s_to_b, b_to_s, s_layer, b_layer), None


class DenseC4:
    name = "c4-dense"
    metric = "routed pairs/sec + MFMA TFLOP/s (% peak), Propagation dense N=4096 D=512 r=64 fwd+bwd"
    workload = "C4-dense Propagation fwd+bwd (all N x N pairs), LowRankBilinearPairwise, softsign, native"
    data = "synthetic (seeded N(0,1) state, unit-norm N(0,1) val rows, default module init)"
    config = {"batch": 16, "nodes": 4096, "dim": 512, "rank": 64}
    traffic_file = "c4_dense_hbm_traffic.json"
    cpu_batch = 4  # CPU baseline sample: 4 of the 16 batch elements

    def edges(self) -> int:
        c = self.config
        return c["batch"] * c["nodes"] * c["nodes"]

    def chunk_batch(self) -> int:
        """Batch elements per launch of the N x N kernels: the library runs
        dense propagation in batch chunks whose edge matrices fit
        jakal_net_native.DENSE_EDGE_BYTES (the whole batch when it fits)."""
        import jakal_net_native as jn

        c = self.config
        B, edge = c["batch"], 4 * c["nodes"] * c["nodes"]
        return B if B * edge <= jn.DENSE_EDGE_BYTES else max(1, min(B, jn.DENSE_EDGE_BYTES // edge))

    def model(self, name):
        c = self.config
        B, N, D, r = (c[x] for x in ("batch", "nodes", "dim", "rank"))
        Bc = self.chunk_batch()  # per launch of the N x N kernels
        dense = {
            "gemm_f32_kernel<dense_scores>": 2.0 * Bc * N * N * r,
            "gemm_f32_kernel<dense_aggregate>": 2.0 * Bc * N * N * D,
            "gemm_f32_kernel<dense_edge_grad>": 2.0 * Bc * N * N * D,
            "gemm_f32_kernel<dense_value_grad>": 2.0 * Bc * N * N * D,
            "gemm_f32_kernel<dense_target_grad>": 2.0 * Bc * N * N * r,
            "gemm_f32_kernel<dense_source_grad>": 2.0 * Bc * N * N * r,
        }
        if name in dense:
            return "mfma", dense[name]
        if name.startswith("dense_compress_backward_kernel"):
            return "hbm", 4.0 * 3 * Bc * N * N  # read G and E, write G_s
        if name.startswith("dense_compress_kernel"):
            return "hbm", 4.0 * 2 * Bc * N * N  # read S, write E
        if name.startswith("dense_colsum_kernel"):
            return "hbm", 4.0 * Bc * N * N
        if name.startswith("gemm_f32_kernel"):
            return "mfma", 2.0 * B * N * D * 2 * r
        return None

    def sparse_bytes(self) -> float:
        # dense: no gathers; the MFMA work is the bound (see roofline)
        c = self.config
        return 4.0 * 6 * c["batch"] * c["nodes"] * c["nodes"]

    def build(self, torch, dev, impl: str = "native", batch: int | None = None):
        from jakal_net import Layer, LowRankBilinearPairwise, Propagation

        B, N, D, r = (self.config[x] for x in ("batch", "nodes", "dim", "rank"))
        B = batch or B
        g = torch.Generator().manual_seed(1004)
        state = torch.randn(B, N, generator=g)
        val = torch.randn(B, N, D, generator=g)
        val = val / val.norm(dim=-1, keepdim=True)
        torch.manual_seed(1004)
        op = Propagation(LowRankBilinearPairwise(D, r), implementation=impl).to(dev)
        return op, Layer(dim=D, num_nodes=N, state=state.to(dev).requires_grad_(True),
                         val=val.to(dev).requires_grad_(True))


class DenseC4Bf16(DenseC4):
    """c4-dense with bf16 layer states and values: the three N x N products
    on bf16 MFMA (the edge matrix rounded to bf16 where it multiplies
    values), the projections on the bf16 projection GEMMs."""

    name = "c4-dense-bf16"
    metric = "routed pairs/sec + MFMA TFLOP/s (% peak), Propagation dense N=4096 D=512 r=64 fwd+bwd, bf16 activations"
    workload = "C4-dense bf16 Propagation fwd+bwd (all N x N pairs), LowRankBilinearPairwise, softsign, bf16 layers, native"
    data = ("synthetic (seeded N(0,1) state, unit-norm N(0,1) val rows, both rounded to bf16; default module "
            "init, fp32 weights)")
    dtype = "bf16"
    traffic_file = "c4_dense_bf16_hbm_traffic.json"
    cpu_batch = 2

    def model(self, name):
        c = self.config
        B, N, D, r = (c[x] for x in ("batch", "nodes", "dim", "rank"))
        Bc = self.chunk_batch()
        dense = {
            "gemm_bf16_kernel<dense_aggregate_bf16>": 2.0 * Bc * N * N * D,
            "gemm_bf16_kernel<dense_edge_grad_bf16>": 2.0 * Bc * N * N * D,
            "gemm_bf16_kernel<dense_value_grad_bf16>": 2.0 * Bc * N * N * D,
        }
        if name in dense:
            return "mfma", dense[name], None, BF16_MFMA_PEAK_TFLOPS
        if name.startswith("gemm_bf16_kernel"):
            return "mfma", 2.0 * B * N * D * 2 * r, None, BF16_MFMA_PEAK_TFLOPS
        return super().model(name)

    def build(self, torch, dev, impl: str = "native", batch: int | None = None):
        from jakal_net import Layer

        op, layer = super().build(torch, dev, impl=impl, batch=batch)
        bf = lambda t: t.detach().bfloat16().requires_grad_(True)  # noqa: E731
        return op, Layer(dim=layer.dim, num_nodes=layer.num_nodes, state=bf(layer.state), val=bf(layer.val))


class DenseCausalC4(DenseC4):
    """C4 shapes with a full causal window (window = N - 1): row i keeps the
    sources j <= i (the causal dense query propagation of
    scripts/progressive_b_example.py:1977-2012, at the C4 size).  The library
    runs it on the dense path with causal K ranges; the algorithmic work is
    the causal half of every N x N product."""

    name = "c4-dense-causal"
    metric = "routed pairs/sec + MFMA TFLOP/s (% peak), Propagation causal dense N=4096 D=512 r=64 fwd+bwd"
    workload = "C4-dense causal (window N-1) SparsePropagation fwd+bwd, LowRankBilinearPairwise, softsign, native"
    traffic_file = "c4_dense_causal_hbm_traffic.json"

    def edges(self) -> int:
        c = self.config
        return c["batch"] * c["nodes"] * (c["nodes"] + 1) // 2

    def model(self, name):
        m = super().model(name)
        if m is not None and m[0] == "mfma" and name.startswith("gemm_f32_kernel<dense_"):
            c = self.config
            N = c["nodes"]
            return m[0], m[1] * (N + 1) / (2 * N), None  # the causal half of the N x N products
        return m

    def build(self, torch, dev, impl: str = "native", batch: int | None = None):
        from jakal_net import Layer, LowRankBilinearPairwise, SparsePropagation

        B, N, D, r = (self.config[x] for x in ("batch", "nodes", "dim", "rank"))
        B = batch or B
        g = torch.Generator().manual_seed(1004)
        state = torch.randn(B, N, generator=g)
        val = torch.randn(B, N, D, generator=g)
        val = val / val.norm(dim=-1, keepdim=True)
        torch.manual_seed(1004)
        op = SparsePropagation(LowRankBilinearPairwise(D, r), sparse_type="window", window=N - 1,
                               implementation=impl).to(dev)
        return op, Layer(dim=D, num_nodes=N, state=state.to(dev).requires_grad_(True),
                         val=val.to(dev).requires_grad_(True))


class TransitionDenseC3:
    name = "c3-transition-dense"
    metric = "routed pairs/sec + MFMA TFLOP/s (% peak), Transition (dense) S->B and B->S N_src=1024 N_dst=256 D=512 fwd+bwd"
    workload = "C3 sizes, dense Transition S->B then B->S fwd+bwd (every destination), LowRankBilinearRoute, softmax routes, native"
    data = "synthetic (seeded N(0,1) states and vals, default module init)"
    config = {"batch": 8, "s_nodes": 1024, "b_nodes": 256, "dim": 512, "rank": 64}
    traffic_file = "c3_transition_dense_hbm_traffic.json"

    def edges(self) -> int:
        c = self.config
        return 2 * c["batch"] * c["s_nodes"] * c["b_nodes"]

    def model(self, name):
        c = self.config
        B, S, Bn, D, r = (c[x] for x in ("batch", "s_nodes", "b_nodes", "dim", "rank"))
        pairs = B * S * Bn  # per direction (both directions route S x B pairs)
        dense = {
            "gemm_f32_kernel<route_logits>": 2.0 * pairs * r,
            "gemm_f32_kernel<route_aggregate>": 2.0 * pairs * D,
            "gemm_f32_kernel<route_edge_grad>": 2.0 * pairs * D,
            "gemm_f32_kernel<route_value_grad>": 2.0 * pairs * D,
            "gemm_f32_kernel<route_source_grad>": 2.0 * pairs * r,
            "gemm_f32_kernel<route_target_grad>": 2.0 * pairs * r,
        }
        if name in dense:
            return "mfma", dense[name]
        if name.startswith("route_dense_compress_backward_kernel"):
            return "hbm", 4.0 * 3 * pairs  # read H and R, write G
        if name.startswith("route_dense_compress_kernel"):
            return "hbm", 4.0 * 2 * pairs
        if name.startswith("route_dense_colsum_kernel"):
            return "hbm", 4.0 * pairs
        if name.startswith("gemm_f32_kernel"):
            return "mfma", 2.0 * B * (S + Bn) / 2 * D * r  # projections, averaged over the two sides
        return None

    def sparse_bytes(self) -> float:
        # dense: no gathers; the route matrices are the bytes that move
        return 4.0 * 6 * self.edges()

    def build(self, torch, dev, impl: str = "native", batch: int | None = None):
        from jakal_net import Layer, LowRankBilinearRoute, Transition

        c = self.config
        B, S, Bn, D, r = (c[x] for x in ("batch", "s_nodes", "b_nodes", "dim", "rank"))
        B = batch or B
        g = torch.Generator().manual_seed(1003)
        s_state, s_val = torch.randn(B, S, generator=g), torch.randn(B, S, D, generator=g)
        b_state, b_val = torch.randn(B, Bn, generator=g), torch.randn(B, Bn, D, generator=g)
        torch.manual_seed(1003)
        s_to_b = Transition(LowRankBilinearRoute(D, D, rank=r), implementation=impl).to(dev)
        b_to_s = Transition(LowRankBilinearRoute(D, D, rank=r), implementation=impl).to(dev)
        s_layer = Layer(dim=D, num_nodes=S, state=s_state.to(dev).requires_grad_(True),
                        val=s_val.to(dev).requires_grad_(True))
        b_layer = Layer(dim=D, num_nodes=Bn, state=b_state.to(dev).requires_grad_(True),
                        val=b_val.to(dev).requires_grad_(True))
        return _TwoWayTransition(torch, s_to_b, b_to_s, s_layer, b_layer), None


class _TwoWayTransition:
    """S->B then B->S routing step with the bench's op/layer interface."""

    def __init__(self, torch, s_to_b, b_to_s, s_layer, b_layer):
        self.torch, self.s_to_b, self.b_to_s, self.s, self.b = torch, s_to_b, b_to_s, s_layer, b_layer

    def zero_grad(self, set_to_none=True):
        self.s_to_b.zero_grad(set_to_none=set_to_none)
        self.b_to_s.zero_grad(set_to_none=set_to_none)
        for layer in (self.s, self.b):
            layer.val.grad = None
            layer.state.grad = None

    def loss_terms(self):
        d1 = self.s_to_b.compute_delta(self.s, self.b)
        d2 = self.b_to_s.compute_delta(self.b, self.s)
        return [d1.delta_state, d1.delta_val, d2.delta_state, d2.delta_val]


class ProgressiveC5:
    """the Progressive-B query-block training step
    (jakal_net.progressive.ProgressiveBStep, the reference's
    ProgressiveBExampleLM glue with low-rank operators) -- prefix encoding
    through S warmup windows, 4 joint blocks (S window, B_cmp -> B_exp expand,
    expanded top-k, B_exp -> S, compress, S -> B_cmp, compressed top-k; each
    update the scaled delta, then tanh / LayerNorm) and S refine windows, then 64
    teacher-forced query slots refined by query transitions and causal query
    propagation, the vocabulary head and the cross entropy -- forward, backward
    and an AdamW update of the fp32 master weights, under bf16 autocast.  The
    unit is processed tokens (prefix + query slots) per second."""

    name = "c5-progressive-b"
    metric = ("tokens/sec, Progressive-B query-block fwd+bwd+AdamW step (vocab 16384, d=512, prefix 512, "
              "4 joint blocks, B_exp 256, B_cmp 64, top-k 16, rank 64, 64 query slots, batch 16), bf16 autocast")
    workload = "C5 Progressive-B query-block training step (fwd+bwd+AdamW), LowRankBilinear operators, native"
    data = "synthetic (uniform random token ids seeded 1005, random init, fp32 master weights)"
    unit = "tokens/s"
    dtype = "bf16 autocast (fp32 master weights; the hot-path ops compute in fp32)"
    config = {"batch": 16, "vocab": 16384, "dim": 512, "prefix": 512, "query": 64, "rank": 64, "topk": 16,
              "blocks": 4, "expanded": 256, "compressed": 64, "s_window": 32}
    traffic_file = "c5_progressive_b_hbm_traffic.json"
    cpu_batch = 2
    eager_only = True

    def edges(self) -> int:  # tokens per step
        c = self.config
        return c["batch"] * (c["prefix"] + c["query"])

    def model(self, name):
        return None  # an end-to-end step: no single roofline

    def sparse_bytes(self):
        return None

    def make_step(self, torch, dev, impl: str = "native", batch: int | None = None, graph: bool = False):
        """graph: the step will be captured into a HIP graph -- AdamW keeps its
        step counts on the device (capturable) and autocast keeps no cast cache."""
        from jakal_net.progressive import ProgressiveBConfig, ProgressiveBStep

        c = self.config
        B = batch or c["batch"]
        cfg = ProgressiveBConfig(vocab=c["vocab"], dim=c["dim"], prefix=c["prefix"], query=c["query"],
                                 rank=c["rank"], topk=c["topk"], blocks=c["blocks"], expanded=c["expanded"],
                                 compressed=c["compressed"], s_window=c["s_window"])
        torch.manual_seed(1005)
        model = ProgressiveBStep(cfg, implementation=impl).to(dev)
        # one fused update kernel per parameter group on the GPU (with device-side step counts)
        fused = dev.type == "cuda"
        opt = torch.optim.AdamW(model.parameters(), lr=1e-4, capturable=graph, fused=fused)
        g = torch.Generator().manual_seed(1005)
        prefix = torch.randint(0, c["vocab"] - 1, (B, c["prefix"]), generator=g).to(dev)
        target = torch.randint(0, c["vocab"] - 1, (B, c["query"]), generator=g).to(dev)
        use_autocast = dev.type == "cuda"  # the CPU baseline runs fp32

        def step() -> None:
            opt.zero_grad(set_to_none=True)
            with torch.autocast(device_type=dev.type, dtype=torch.bfloat16, enabled=use_autocast,
                                cache_enabled=not graph):
                loss = model(prefix, target)
            loss.backward()
            opt.step()
        return step


WORKLOADS = {w.name: w for w in (TopkC4(), TopkC4Bf16(), WindowC2(), TransitionC3(), DenseC4(), DenseC4Bf16(),
                                 DenseCausalC4(), TransitionDenseC3(), ProgressiveC5())}


def capture_step(torch, step):
    """Capture one call of `step` into a HIP graph and return its replay.
    Two warm-up calls run first on a side stream (default priority), so lazy
    initialisation happens outside the capture."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    return graph.replay


def workload_step(wl, torch, dev, impl: str = "native", batch: int | None = None, graph: bool = False):
    """The timed step of a workload: its own make_step, or forward+backward of its operator."""
    if hasattr(wl, "make_step"):
        return wl.make_step(torch, dev, impl, batch, graph=graph)
    op, layer = wl.build(torch, dev, impl=impl, batch=batch)
    return _make_step(torch, op, layer)

COPY_BYTES = 1 << 30


def calibrate_copy(torch) -> int:
    """Five launches of a plain device-to-device copy of COPY_BYTES (read COPY_BYTES,
    write COPY_BYTES); the per-dispatch FETCH_SIZE / WRITE_SIZE a profiler reads
    for it scale those counters to bytes."""
    src = torch.ones(COPY_BYTES // 4, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": COPY_BYTES, "copy_bytes_written": COPY_BYTES, "launches": 5}))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="c4-topk")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--select-mode", choices=["split-f16", "f32"], default="split-f16",
                    help="score arithmetic of the top-k select (library default: split-f16)")
    ap.add_argument("--gemm-tile", type=int, choices=[0, 64, 128], default=0,
                    help="force the GEMM workgroup tile (0: chosen per call)")
    ap.add_argument("--eager", action="store_true",
                    help="time eager steps only (default for the operator workloads: time replays of the step "
                         "captured into one HIP graph, torch.cuda.CUDAGraph, after timing the same number of "
                         "eager steps with per-kernel HIP events)")
    ap.add_argument("--no-alone", action="store_true",
                    help="skip the serial pass (side streams off) that times each kernel alone; for profiler "
                         "runs that should see the timed steps only")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain device copy of known size (scale for HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path.",
              file=sys.stderr)
        return 2

    import torch

    if args.calibrate_copy:
        return calibrate_copy(torch)

    import jakal_net_native as jn

    jn.set_gemm_tile(args.gemm_tile)
    jn.set_select_mode(jn.SELECT_SPLIT_F16 if args.select_mode == "split-f16" else jn.SELECT_F32)
    wl = WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    # C5's full-size step is timed eagerly: capturing it into a HIP graph after
    # eager steps has ended in a host segmentation fault inside torch's
    # capture_end, whose cause is not known
    use_graph = not args.eager and not getattr(wl, "eager_only", False)
    step = workload_step(wl, torch, dev, graph=use_graph)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    def timed(fn):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record()
        for _ in range(args.steps):
            fn()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / args.steps, time.perf_counter() - t0

    # eager steps with the library's per-kernel HIP events on the launch stream
    jn.profile_enable(True)
    eager_ms, wall = timed(step)
    prof = jn.profile_collect()
    # the same kernels once more with the side streams off: each kernel alone
    # (the timings above include the overlap of the two streams' kernels)
    jn.set_side_streams(False)
    alone_steps = 0 if args.no_alone else max(1, min(args.steps, 5))
    for _ in range(alone_steps):
        step()
    torch.cuda.synchronize()
    prof_alone = jn.profile_collect() if alone_steps else {}
    jn.profile_enable(False)
    jn.set_side_streams(True)
    ms_per_step = eager_ms
    graph_info = None
    if use_graph:
        replay = capture_step(torch, step)
        for _ in range(args.warmup):
            replay()
        ms_per_step, wall = timed(replay)
        graph_info = {"eager_ms_per_step": round(eager_ms, 5), "eager_value": wl.edges() / (eager_ms / 1e3),
                      "note": "value and ms_per_step time back-to-back replays of one captured forward+backward "
                              "step (every kernel runs each replay); the kernel table and roofline come from the "
                              "eager steps timed just before with HIP events on the launch stream (same kernels)"}
    E = wl.edges()
    value = E / (ms_per_step / 1e3)

    kernels = {}
    for name, (count, total_ms) in sorted(prof.items(), key=lambda kv: -kv[1][1]):
        avg_ms = total_ms / count
        entry = {"launches_per_step": count / args.steps, "avg_ms": round(avg_ms, 5),
                 "ms_per_step": round(total_ms / args.steps, 5)}
        if name in prof_alone:
            entry["avg_ms_alone"] = round(prof_alone[name][1] / prof_alone[name][0], 5)
        x3 = name.startswith("gemm_x3_kernel")
        # fp32 GEMMs on three-term bf16 splits: the work of the same use on fp32 MFMA, against their own bound
        model = wl.model(name.replace("gemm_x3_kernel", "gemm_f32_kernel", 1) if x3 else name)
        if model is not None and x3:
            model = (model[0], model[1], None, X3_MFMA_PEAK_TFLOPS)
        if model is not None:
            bound, work = model[0], model[1]
            if bound == "hbm":
                # HBM roofline on compulsory bytes; the algorithmic (every operand
                # once per use) rate is reported beside it as an L2-side figure
                compulsory = model[2] if len(model) > 2 and model[2] is not None else work
                achieved = compulsory / (avg_ms / 1e3) / 1e9
                entry.update(bound="hbm", compulsory_bytes=compulsory, achieved_GBps=round(achieved, 1),
                             frac=round(achieved / HBM_PEAK_GBS, 4), algorithmic_bytes=work,
                             l2_side_GBps=round(work / (avg_ms / 1e3) / 1e9, 1))
                if "avg_ms_alone" in entry:
                    alone = compulsory / (entry["avg_ms_alone"] / 1e3) / 1e9
                    entry.update(achieved_GBps_alone=round(alone, 1), frac_alone=round(alone / HBM_PEAK_GBS, 4))
            else:
                achieved = work / (avg_ms / 1e3) / 1e12
                peak = model[3] if len(model) > 3 else FP32_MFMA_PEAK_TFLOPS
                entry.update(bound="mfma", flops=work, achieved_TFLOPs=round(achieved, 2), peak_TFLOPs=peak,
                             frac=round(achieved / peak, 4))
                if name.startswith("lowrank_topk_select_kernel"):
                    if getattr(wl, "dtype", "f32") == "bf16":
                        entry.update(arith="bf16 MFMA (v_mfma_f32_16x16x32_bf16), fp32 accumulate")
                    elif args.select_mode == "split-f16":
                        # flops count fp32-equivalent score products; the MFMA pipe runs
                        # SPLIT_PRODUCTS fp16 products for each
                        f16 = SPLIT_PRODUCTS * achieved
                        entry.update(arith="split-fp16 MFMA (hi.hi + hi.lo + lo.hi), fp32 accumulate",
                                     mfma_f16_TFLOPs=round(f16, 2),
                                     mfma_f16_frac=round(f16 / FP16_MFMA_PEAK_TFLOPS, 4))
                    else:
                        entry.update(arith="fp32 MFMA")
                if x3:
                    entry.update(arith="fp32 operands as three bf16 terms, six bf16 MFMA products, fp32 accumulate",
                                 fp32_equivalent_frac=round(achieved / FP32_MFMA_PEAK_TFLOPS, 4))
        kernels[name] = entry

    # HBM-side bytes per launch measured by rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    # of this same command (scaled by a copy kernel of known size), when present
    measured = {}
    traffic_file = ROOT / "profiles" / wl.traffic_file
    if traffic_file.exists():
        measured = json.loads(traffic_file.read_text()).get("kernels", {})
        # timing names whose kernel function has another name in the rocprofv3 summaries
        for name, func in (("route_gather_kernel", "cols_gather_kernel"),
                           ("unit_scale_backward_kernel", "unit_scale_kernel")):
            if name not in measured and func in measured:
                measured[name] = measured[func]
    for name, entry in kernels.items():
        if name in measured:
            entry["traffic_bytes"] = measured[name]["traffic_bytes"]
            entry["traffic_GBps"] = round(measured[name]["traffic_bytes"] / (entry["avg_ms"] / 1e3) / 1e9, 1)

    # step-level HBM-side traffic: every kernel's measured bytes per launch
    # (rocprofv3 FETCH_SIZE + WRITE_SIZE of this workload) times its launches
    # per step, over the step time; and the compulsory bytes of the modelled
    # HBM-bound kernels over the same time
    hbm = None
    if measured:
        traffic = sum(measured[n]["traffic_bytes"] * e["launches_per_step"] for n, e in kernels.items()
                      if n in measured)
        missing = sorted(n for n in kernels if n not in measured)
        compulsory = sum(e["compulsory_bytes"] * e["launches_per_step"] for e in kernels.values()
                         if e.get("bound") == "hbm")
        traffic_json = json.loads(traffic_file.read_text())
        hbm = {
            "measured_bytes_per_step": traffic,
            "measured_GBps": round(traffic / (ms_per_step / 1e3) / 1e9, 1),
            "measured_frac": round(traffic / (ms_per_step / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
            "compulsory_bytes_per_step": compulsory,
            "compulsory_GBps": round(compulsory / (ms_per_step / 1e3) / 1e9, 1),
            "compulsory_frac": round(compulsory / (ms_per_step / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
            "counter_source": f"profiles/{wl.traffic_file} (commit {traffic_json.get('commit')})",
            "kernels_without_counters": missing,
            "note": "measured: rocprofv3 FETCH_SIZE + WRITE_SIZE bytes per launch (L2-to-fabric traffic, scaled by "
                    "a device copy of known size) x launches per step / ms_per_step; compulsory: each distinct "
                    "input row and output of the HBM-bound kernels once",
        }

    modeled = [(n, e) for n, e in kernels.items() if "bound" in e]
    dom_name, dom = max(modeled or list(kernels.items()), key=lambda ne: ne[1]["ms_per_step"])
    if not modeled:  # an end-to-end step: the hottest kernel, without a roofline
        roofline = {"kernel": dom_name, "bound": None, "achieved": None, "peak": None, "unit": None, "frac": None,
                    "traffic": dom.get("traffic_bytes"),
                    "note": "end-to-end step of many small operators; per-kernel figures under 'kernels'"}
    elif dom["bound"] == "hbm":
        roofline = {"kernel": dom_name, "bound": "hbm", "achieved": dom["achieved_GBps"], "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": dom["frac"], "traffic": dom.get("traffic_bytes")}
    else:
        roofline = {"kernel": dom_name, "bound": "mfma", "achieved": dom["achieved_TFLOPs"],
                    "peak": dom["peak_TFLOPs"], "unit": "TFLOP/s", "frac": dom["frac"],
                    "traffic": dom.get("traffic_bytes")}
        if "arith" in dom:
            roofline["arith"] = dom["arith"]

    sparse_rate = (None if wl.sparse_bytes() is None
                   else round(wl.sparse_bytes() / (ms_per_step / 1e3) / 1e9, 1))
    sparse_note = None
    if sparse_rate is not None:
        sparse_note = ("BASELINE's sparse-phase bytes (every operand once per use, no cache reuse) / ms_per_step: "
                       "an algorithmic rate, not bytes moved")
        if sparse_rate > HBM_PEAK_GBS:
            sparse_note += (f"; above the {HBM_PEAK_GBS:.0f} GB/s HBM peak, so the step is not HBM-bound at this "
                            "shape (the gathers re-read rows from L2); hbm_measured_GBps is the bytes moved")
    result = {
        "metric": wl.metric,
        "value": value,
        "unit": getattr(wl, "unit", "routed pairs/s"),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": getattr(wl, "dtype", "f32"),
        "data": wl.data,
        "config": {"workload": wl.workload, **wl.config},
        "hbm_measured_GBps": None if hbm is None else hbm["measured_GBps"],
        "hbm_frac": None if hbm is None else hbm["measured_frac"],
        "hbm": hbm,
        "sparse_phase_algorithmic_GBps": sparse_rate,
        "sparse_phase_note": sparse_note,
        "roofline": roofline,
        "kernels": kernels,
        "wall_s_timed": round(wall, 3),
        "graph": graph_info,
        "device": torch.cuda.get_device_name(0),
    }
    if not args.no_cpu_baseline:
        del step
        torch.cuda.empty_cache()
    result["cpu_baseline"] = None if args.no_cpu_baseline else cpu_baseline(wl, torch)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
