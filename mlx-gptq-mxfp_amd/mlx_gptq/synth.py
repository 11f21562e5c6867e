"""Seeded synthetic calibration workloads shaped like the benchmark configs.

No checkpoints or datasets are available offline, so the solver is measured
on synthetic data of the real shapes: lognormal per-channel activation
scales with outlier channels, N(0, sigma) bf16 weights, and for the MoE
layer a top-k router with a Zipf-like expert bias. Generation is seeded and
deterministic; it is setup work, never part of a timed region.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass
class MoELayer:
    """Config-4 style routed-expert layer, device resident."""

    X: torch.Tensor          # bf16 [tokens, hidden] hidden states
    row_index: torch.Tensor  # int32 [tokens*top_k] token id per assignment, grouped by expert
    offsets: list            # python ints [E+1]: expert e owns row_index[offsets[e]:offsets[e+1]]
    Y: torch.Tensor          # bf16 [tokens*top_k, inter] down-proj inputs, same order
    W_gate_up: torch.Tensor  # bf16 [E, 2*inter, hidden] (gate rows first, then up)
    W_down: torch.Tensor     # bf16 [E, hidden, inter]
    n_empty: int             # the last n_empty experts receive no tokens

    @property
    def experts(self) -> int:
        return self.W_gate_up.shape[0]

    def counts(self) -> list:
        return [self.offsets[e + 1] - self.offsets[e] for e in range(self.experts)]


def _hidden_states(n_tokens: int, hidden: int, device, chunk: int = 65536,
                   sigma: float = 1.0, outlier_frac: float = 0.0, outlier_mult: float = 1.0,
                   seed: int = 17) -> torch.Tensor:
    """N(0,1) rows scaled per channel by exp(N(0, sigma)); a seeded subset of
    channels multiplied by outlier_mult. Chunk c uses generator seed + c."""
    g = torch.Generator().manual_seed(seed - 1)
    scale = torch.exp(torch.randn(hidden, generator=g) * sigma)
    n_out = int(round(outlier_frac * hidden))
    if n_out:
        scale[torch.randperm(hidden, generator=g)[:n_out]] *= outlier_mult
    scale = scale.to(device)
    out = torch.empty(n_tokens, hidden, dtype=torch.bfloat16, device=device)
    for c, a in enumerate(range(0, n_tokens, chunk)):
        b = min(a + chunk, n_tokens)
        gc = torch.Generator(device=device).manual_seed(seed + c)
        x = torch.randn(b - a, hidden, generator=gc, device=device)
        out[a:b] = (x * scale).to(torch.bfloat16)
    return out


@torch.no_grad()
def moe_layer(experts: int = 128, hidden: int = 2048, inter: int = 768, tokens: int = 131072,
              top_k: int = 8, n_empty: int = 4, w_std: float = 0.02, device="cuda:0",
              seed: int = 17) -> MoELayer:
    """Qwen3-30B-A3B-shaped MoE layer (benchmark config 4).

    Router logits X.R (R ~ N(0, 0.05)) plus a Zipf(1.1) expert bias
    -1.1*ln(rank) over a seeded rank permutation; the last `n_empty` experts
    get bias -inf (forced empty). top_k of the logits (= of the softmax).
    Down-proj inputs are bf16(SiLU(x W_g^T) * (x W_u^T)) with the unquantized
    expert weights, as the layer's own forward would produce them.
    """
    X = _hidden_states(tokens, hidden, device, sigma=1.0, seed=seed)
    g = torch.Generator().manual_seed(seed + 1000)
    R = (torch.randn(hidden, experts, generator=g) * 0.05).to(device)
    rank = torch.randperm(experts, generator=g).to(torch.float32) + 1.0
    bias = -1.1 * torch.log(rank)
    if n_empty:
        bias[experts - n_empty:] = -math.inf
    bias = bias.to(device)
    logits = torch.empty(tokens, experts, device=device)
    for a in range(0, tokens, 16384):
        b = min(a + 16384, tokens)
        logits[a:b] = X[a:b].float() @ R + bias
    top = logits.topk(top_k, dim=1).indices.reshape(-1)
    del logits
    token = torch.arange(tokens, device=device).repeat_interleave(top_k)
    order = torch.argsort(top, stable=True)
    row_index = token[order].to(torch.int32).contiguous()
    counts = torch.bincount(top, minlength=experts)
    offsets = [0] + torch.cumsum(counts, 0).tolist()

    gw = torch.Generator(device=device).manual_seed(seed + 2000)
    W_gu = (torch.randn(experts, 2 * inter, hidden, generator=gw, device=device) * w_std).to(torch.bfloat16)
    W_dn = (torch.randn(experts, hidden, inter, generator=gw, device=device) * w_std).to(torch.bfloat16)

    Y = torch.empty(offsets[-1], inter, dtype=torch.bfloat16, device=device)
    for e in range(experts):
        a, b = offsets[e], offsets[e + 1]
        if a == b:
            continue
        xe = X.index_select(0, row_index[a:b].long())
        gate = F.linear(xe, W_gu[e, :inter])
        up = F.linear(xe, W_gu[e, inter:])
        Y[a:b] = (F.silu(gate.float()) * up.float()).to(torch.bfloat16)
    return MoELayer(X, row_index, offsets, Y, W_gu, W_dn, n_empty)


@torch.no_grad()
def dense_linear(rows: int, cols: int, tokens: int, w_std: float = 0.02, sigma: float = 1.0,
                 outlier_frac: float = 0.0, outlier_mult: float = 1.0, device="cuda:0", seed: int = 17):
    """(W bf16 [1, rows, cols], X bf16 [tokens, cols]) for a dense linear."""
    X = _hidden_states(tokens, cols, device, sigma=sigma, outlier_frac=outlier_frac,
                       outlier_mult=outlier_mult, seed=seed)
    gw = torch.Generator(device=device).manual_seed(seed + 3000)
    W = (torch.randn(1, rows, cols, generator=gw, device=device) * w_std).to(torch.bfloat16)
    return W, X


@torch.no_grad()
def swiglu_inputs(n_tokens: int, channels: int, device, sigma: float = 1.0, seed: int = 29,
                  chunk: int = 8192) -> torch.Tensor:
    """Down-projection inputs bf16(SiLU(a) * b) with a, b ~ N(0, 1), each
    channel scaled by exp(N(0, sigma)); chunk c uses generator seed + c."""
    g = torch.Generator().manual_seed(seed - 1)
    scale = torch.exp(torch.randn(channels, generator=g) * sigma).to(device)
    out = torch.empty(n_tokens, channels, dtype=torch.bfloat16, device=device)
    for c, a in enumerate(range(0, n_tokens, chunk)):
        b = min(a + chunk, n_tokens)
        gc = torch.Generator(device=device).manual_seed(seed + c)
        x = torch.randn(b - a, channels, generator=gc, device=device)
        y = torch.randn(b - a, channels, generator=gc, device=device)
        out[a:b] = (F.silu(x) * y * scale).to(torch.bfloat16)
        del x, y
    return out


@dataclass
class DenseMatrix:
    """One weight matrix of a dense layer and how the benchmark solves it."""

    name: str
    W: torch.Tensor   # bf16 [1, out, in]
    inp: str          # key of its calibration input in DenseLayer.inputs
    solve: dict       # solve_gptq keyword arguments (bits, group_size, mode, ...)
    pack_bits: int


@dataclass
class DenseLayer:
    name: str
    inputs: dict      # key -> bf16 [tokens, in] calibration rows
    mats: list        # DenseMatrix, in solve order

    @property
    def elements(self) -> int:
        return sum(int(m.W.numel()) for m in self.mats)


@torch.no_grad()
def dense_config(cfg: int, device="cuda:0") -> DenseLayer:
    """BASELINE configs 1, 2, 3 and 5 (dense linears / MLPs)."""
    def w(rows, cols, std, seed):
        gw = torch.Generator(device=device).manual_seed(seed)
        return (torch.randn(1, rows, cols, generator=gw, device=device) * std).to(torch.bfloat16)

    if cfg == 1:
        X = _hidden_states(8192, 2048, device, outlier_frac=0.01, outlier_mult=20.0, seed=17)
        return DenseLayer("cfg1 single Linear [2048,2048], affine 4-bit GPTQ (G=64, block 128, MSE clip)",
                          {"x": X}, [DenseMatrix("linear", w(2048, 2048, 0.02, 3017), "x",
                                                 dict(bits=4, group_size=64, mode="affine"), 4)])
    if cfg == 2:
        X = _hidden_states(32768, 4096, device, outlier_frac=0.005, outlier_mult=30.0, seed=17)
        return DenseLayer("cfg2 Llama-3-8B q_proj [4096,4096], MXFP4 groupwise GPTQ",
                          {"x": X}, [DenseMatrix("q_proj", w(4096, 4096, 0.02, 3017), "x",
                                                 dict(bits=4, group_size=32, mode="mxfp4",
                                                      mxfp_algorithm="groupwise"), 4)])
    if cfg == 3:
        X = _hidden_states(65536, 4096, device, outlier_frac=0.01, outlier_mult=20.0, seed=17)
        Xd = swiglu_inputs(65536, 14336, device, seed=29)
        kw = dict(bits=8, group_size=32, mode="mxfp8", mxfp_algorithm="groupwise")
        return DenseLayer("cfg3 Llama-3-8B MLP: up [14336,4096] + down [4096,14336], MXFP8 groupwise GPTQ",
                          {"x": X, "act": Xd},
                          [DenseMatrix("up_proj", w(14336, 4096, 0.015, 3017), "x", kw, 8),
                           DenseMatrix("down_proj", w(4096, 14336, 0.015, 3018), "act", kw, 8)])
    if cfg == 5:
        X = _hidden_states(524288, 5120, device, outlier_frac=0.01, outlier_mult=25.0, seed=17)
        Xd = swiglu_inputs(524288, 25600, device, seed=29)
        kw = dict(bits=4, group_size=32, mode="mxfp4", mxfp_algorithm="safe-scale-search")
        return DenseLayer("cfg5 Qwen3-32B MLP: gate, up [25600,5120] + down [5120,25600], MXFP4 "
                          "safe-scale-search GPTQ",
                          {"x": X, "act": Xd},
                          [DenseMatrix("gate_proj", w(25600, 5120, 0.015, 3017), "x", kw, 4),
                           DenseMatrix("up_proj", w(25600, 5120, 0.015, 3018), "x", kw, 4),
                           DenseMatrix("down_proj", w(5120, 25600, 0.015, 3019), "act", kw, 4)])
    raise ValueError(f"no dense benchmark config {cfg} (1, 2, 3 or 5; config 4 is moe_layer)")
