"""Routed capture (capture.RoutedStash / capture.ExpertCapture) against what
the experts' F.linear calls actually receive.

The ground truth is taken the way the reference's own capture takes it
(mlx_gptq/capture.py:192-207): a TorchFunctionMode that records the input of
every F.linear whose weight is an expert slice. The routed capture never
copies per-expert rows for the input projections, so its rows are checked
against those recordings (as multisets: the row order inside an expert
differs), its down_proj rows in arrival order, and on the GPU its grouped
Hessians against fp64 X^T X of the recorded rows (1e-5 relative Frobenius,
the Hessian bar).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch.overrides import TorchFunctionMode

from mlx_gptq import capture

transformers = pytest.importorskip("transformers")
from transformers import Qwen3MoeConfig  # noqa: E402
from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock  # noqa: E402


class _Recorder(TorchFunctionMode):
    """rows[(param name, expert)] = inputs of F.linear on that expert slice."""

    def __init__(self, block):
        super().__init__()
        self.ptr = {}
        for pname, p in block.experts.named_parameters(recurse=False):
            for e in range(p.shape[0]):
                self.ptr[p.data_ptr() + e * p.stride(0) * p.element_size()] = (pname, e)
        self.rows = {}

    def __torch_function__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if func is F.linear and len(args) >= 2 and isinstance(args[1], torch.Tensor):
            hit = self.ptr.get(args[1].data_ptr())
            if hit is not None:
                self.rows.setdefault(hit, []).append(args[0].detach().to(torch.bfloat16).cpu())
        return func(*args, **kwargs)


def _block(E=8, k=2, hidden=64, inter=32, seed=0, device="cpu", dtype=torch.float32):
    cfg = Qwen3MoeConfig(hidden_size=hidden, moe_intermediate_size=inter, num_experts=E,
                         num_experts_per_tok=k, norm_topk_prob=True)
    torch.manual_seed(seed)
    blk = Qwen3MoeSparseMoeBlock(cfg)
    for p in blk.parameters():
        torch.nn.init.normal_(p, std=0.2)
    return blk.to(device=device, dtype=dtype)


def _run(blk, batches, device="cpu", dtype=torch.float32):
    cap = capture.ExpertCapture(blk)
    rec = _Recorder(blk)
    g = torch.Generator().manual_seed(1)
    hidden = blk.experts.gate_up_proj.shape[-1]
    with torch.no_grad(), cap, rec:
        for shape in batches:
            blk(torch.randn(*shape, hidden, generator=g).to(device=device, dtype=dtype))
    return cap, rec


def _sorted_rows(x: torch.Tensor) -> np.ndarray:
    a = x.float().numpy().astype(np.float64)
    if a.shape[0] == 0:
        return a
    return a[np.lexsort(a.T[::-1])]


def _recorded(rec, pname, e, C):
    parts = rec.rows.get((pname, e), [])
    return torch.cat(parts) if parts else torch.zeros(0, C, dtype=torch.bfloat16)


def test_routed_rows_are_the_rows_each_expert_received():
    blk = _block()
    cap, rec = _run(blk, [(2, 5), (1, 7), (3, 4)])
    gu, dn = cap.stashes["experts.gate_up_proj"], cap.stashes["experts.down_proj"]
    assert gu.rows == 10 + 7 + 12  # the block input, stored once
    counts = gu.token_counts()
    assert counts.sum() == 2 * (10 + 7 + 12)
    for e in range(8):
        want = _recorded(rec, "gate_up_proj", e, 64)
        got = gu.expert_rows(e)
        assert got.dtype == torch.bfloat16 and got.shape == want.shape
        np.testing.assert_array_equal(_sorted_rows(got), _sorted_rows(want))
        # down_proj inputs exist per expert only: stored in arrival order
        want_d = _recorded(rec, "down_proj", e, 32)
        assert torch.equal(dn.expert_rows(e), want_d)
    stats = cap.expert_token_stats()
    assert stats["experts.gate_up_proj"][2] == counts.max()
    cap.check_capture_happened()


def test_out_of_range_expert_ids_are_dropped_and_spans_offset():
    st = capture.RoutedStash("s", 4, 3)
    x = torch.arange(20, dtype=torch.float32).reshape(5, 4)
    ti = torch.tensor([[0, 3], [1, -1], [2, 0], [3, 3], [1, 2]])
    st.add_routed(x, ti)
    st.add_rows(1, torch.ones(2, 4))
    X, off, ri = st.plan()
    # expert 0: tokens 0, 2; expert 1: token 1, token 4, the two added rows
    # (buffer rows 5, 6); expert 2: tokens 2, 4; ids 3 and -1 go nowhere
    assert off.tolist() == [0, 2, 6, 8]
    assert sorted(ri[off[0]:off[1]].tolist()) == [0, 2]
    assert sorted(ri[off[1]:off[2]].tolist()) == [1, 4, 5, 6]
    assert sorted(ri[off[2]:off[3]].tolist()) == [2, 4]
    assert X.shape == (7, 4) and X.dtype == torch.bfloat16
    assert torch.equal(X[:5], x.to(torch.bfloat16))


def test_add_rows_counts_and_expert_range():
    st = capture.RoutedStash("s", 4, 3)
    st.add_rows(2, torch.ones(3, 4))
    st.add_routed(torch.zeros(2, 4), torch.tensor([[0], [2]]))
    assert st.token_counts().tolist() == [1, 0, 4]
    assert torch.equal(st.expert_rows(2)[:3], torch.ones(3, 4, dtype=torch.bfloat16))
    with pytest.raises(IndexError):
        st.add_rows(3, torch.ones(1, 4))
    with pytest.raises(RuntimeError):
        st.add_rows(0, torch.ones(1, 5))
    with pytest.raises(ValueError):
        st.add_routed(torch.zeros(2, 4), torch.zeros(3, dtype=torch.int64))


def test_inputs_are_copied():
    x = torch.ones(3, 4)
    st = capture.Stash("a", 4)
    st.add(x)
    rs = capture.RoutedStash("b", 4, 2)
    rs.add_routed(x, torch.tensor([[0], [1], [0]]))
    x.fill_(7.0)
    assert bool((st.chunks[0] == 1).all()) and bool((rs.expert_rows(0) == 1).all())


class _NoTopK(torch.nn.Module):
    """A fused expert module that routes internally (no top_k_index
    argument): capture falls back to recording F.linear inputs per slice."""

    def __init__(self, E=4, hidden=32, inter=16):
        super().__init__()
        g = torch.Generator().manual_seed(5)
        self.gate_up_proj = torch.nn.Parameter(torch.randn(E, 2 * inter, hidden, generator=g) * 0.2)
        self.down_proj = torch.nn.Parameter(torch.randn(E, hidden, inter, generator=g) * 0.2)

    def forward(self, hidden_states):
        out = torch.zeros_like(hidden_states)
        route = hidden_states[:, 0].abs().mul(100).long() % self.gate_up_proj.shape[0]
        for e in range(self.gate_up_proj.shape[0]):
            idx = torch.nonzero(route == e).flatten()
            if idx.numel() == 0:
                continue
            gu = F.linear(hidden_states[idx], self.gate_up_proj[e])
            gate, up = gu.chunk(2, dim=-1)
            out[idx] = F.linear(F.silu(gate) * up, self.down_proj[e])
        return out


def test_fallback_without_top_k_records_slice_inputs():
    m = _NoTopK()
    cap = capture.ExpertCapture(m)
    rec = _Recorder(type("B", (), {"experts": m})())
    g = torch.Generator().manual_seed(2)
    with torch.no_grad(), cap, rec:
        for _ in range(2):
            m(torch.randn(9, 32, generator=g))
    for key, pname, C in (("gate_up_proj", "gate_up_proj", 32), ("down_proj", "down_proj", 16)):
        st = cap.stashes[key]
        for e in range(4):
            assert torch.equal(st.expert_rows(e), _recorded(rec, pname, e, C))


def test_backfill_unrouted_experts():
    blk = _block(E=8, k=2)
    gate_fwd = blk.gate.forward

    def never_seven(h):  # the router never picks expert 7
        logits, _, _ = gate_fwd(h)
        masked = logits.clone()
        masked[:, 7] = -float("inf")
        probs = torch.softmax(masked, dim=-1, dtype=torch.float)
        vals, idx = torch.topk(probs, 2, dim=-1)
        return logits, (vals / vals.sum(-1, keepdim=True)).to(logits.dtype), idx

    blk.gate.forward = never_seven
    cap = capture.ExpertCapture(blk)
    g = torch.Generator().manual_seed(3)
    xs = [torch.randn(1, 100, 64, generator=g), torch.randn(2, 10, 64, generator=g)]
    with torch.no_grad(), cap:
        for x in xs:
            blk(x)
    gu, dn = cap.stashes["experts.gate_up_proj"], cap.stashes["experts.down_proj"]
    assert gu.token_counts()[7] == 0 and dn.token_counts()[7] == 0
    assert cap.backfill_unrouted_experts() == {"experts": [7]}
    # the sample: 64 evenly spaced rows of a batch with more than 64 (capture.py:52-63)
    rows = [x.reshape(-1, 64) for x in xs]
    sample = torch.cat([rows[0][torch.linspace(0, 99, 64).long()], rows[1]]).to(torch.bfloat16)
    assert torch.equal(gu.expert_rows(7), sample)
    # down inputs: the sample in the weights' dtype through expert 7's own
    # gate/up projections (capture.py:300-306), stored as bf16
    w = blk.experts.gate_up_proj[7].detach()
    gate, up = F.linear(sample.to(w.dtype), w).chunk(2, dim=-1)
    assert torch.equal(dn.expert_rows(7), (F.silu(gate) * up).to(torch.bfloat16))
    assert cap.fallback_experts == {"experts.gate_up_proj::e7": "all_expert_inputs",
                                    "experts.down_proj::e7": "all_expert_inputs"}
    assert cap.backfill_unrouted_experts() == {}


def test_group_size_skip_and_no_capture_error():
    blk = _block(hidden=48, inter=32)
    cap = capture.ExpertCapture(blk, group_size=32)
    assert cap.skipped == ["experts.gate_up_proj"] and list(cap.params) == ["experts.down_proj"]
    with pytest.raises(RuntimeError, match="No tokens captured"):
        cap.check_capture_happened()


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
def test_hessians_need_a_hip_device():
    st = capture.RoutedStash("s", 32, 2)
    st.add_routed(torch.ones(4, 32), torch.tensor([[0], [1], [0], [1]]))
    with pytest.raises(RuntimeError, match="HIP devices only"):
        st.hessians("cpu")


# ---------------------------------------------------------------------------
# GPU: grouped Hessians of the captured rows
# ---------------------------------------------------------------------------
def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.double() - b).norm() / b.norm().clamp(min=1e-300))


@pytest.mark.gpu
def test_gpu_routed_hessians_match_recorded_rows():
    dev = torch.device("cuda", 0)
    blk = _block(E=16, k=4, hidden=256, inter=128, device=dev, dtype=torch.bfloat16)
    cap, rec = _run(blk, [(4, 96), (2, 77), (1, 300)], device=dev, dtype=torch.bfloat16)
    for key, pname, C in (("experts.gate_up_proj", "gate_up_proj", 256),
                          ("experts.down_proj", "down_proj", 128)):
        H = cap.hessians(key, dev)
        assert H.shape == (16, C, C) and H.dtype == torch.float32
        for e in range(16):
            x = _recorded(rec, pname, e, C).double()
            ref = x.T @ x
            if x.shape[0] == 0:
                assert bool((H[e] == 0).all())
            else:
                assert _rel(H[e].cpu(), ref) < 1e-5, (key, e)
        sub = cap.stashes[key].hessians(dev, range(3, 9))
        assert _rel(sub.cpu(), H[3:9].cpu().double()) < 1e-6
        assert _rel(cap.stashes[key].hessian(5, dev).cpu(), H[5].cpu().double()) < 1e-6


@pytest.mark.gpu
def test_gpu_routed_stash_empty_experts_and_cpu_rows():
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(9)
    st = capture.RoutedStash("s", 64, 6)
    xs = [torch.randn(50, 64, generator=g) for _ in range(3)]
    tis = [torch.randint(0, 4, (50, 2), generator=g) for _ in range(3)]
    for x, ti in zip(xs, tis):
        st.add_routed(x, ti)  # rows captured on the CPU, moved once by hessians()
    H = st.hessians(dev)
    X = torch.cat(xs).to(torch.bfloat16).double()
    T = torch.cat(tis)
    for e in range(6):
        # a row routed twice to one expert counts twice, as the eager loop's
        # torch.where over the one-hot top-k mask lists it twice
        w = (T == e).sum(dim=1).double()
        ref = (X * w[:, None]).T @ X
        if e >= 4:
            assert bool((H[e] == 0).all())
        else:
            assert _rel(H[e].cpu(), ref) < 1e-5


class _SeparateGateUp(torch.nn.Module):
    """Fused experts with separate 3D gate_proj / up_proj parameters, routed
    internally (no top_k_index): both slices' F.linear calls see the same
    input tensor, which must be stored once per expert."""

    def __init__(self, E=4, hidden=32, inter=16):
        super().__init__()
        g = torch.Generator().manual_seed(6)
        self.gate_proj = torch.nn.Parameter(torch.randn(E, inter, hidden, generator=g) * 0.2)
        self.up_proj = torch.nn.Parameter(torch.randn(E, inter, hidden, generator=g) * 0.2)
        self.down_proj = torch.nn.Parameter(torch.randn(E, hidden, inter, generator=g) * 0.2)

    def forward(self, hidden_states):
        out = torch.zeros_like(hidden_states)
        route = hidden_states[:, 0].abs().mul(100).long() % self.gate_proj.shape[0]
        for e in range(self.gate_proj.shape[0]):
            idx = torch.nonzero(route == e).flatten()
            if idx.numel() == 0:
                continue
            x = hidden_states[idx]
            h = F.silu(F.linear(x, self.gate_proj[e])) * F.linear(x, self.up_proj[e])
            out[idx] = F.linear(h, self.down_proj[e])
        return out


def test_separate_gate_up_fallback_stores_each_row_once():
    m = _SeparateGateUp()
    cap = capture.ExpertCapture(m)
    rec = _Recorder(type("B", (), {"experts": m})())
    g = torch.Generator().manual_seed(4)
    with torch.no_grad(), cap, rec:
        for _ in range(3):
            m(torch.randn(11, 32, generator=g))
    st = cap.stashes["gate_proj"]
    assert st is cap.stashes["up_proj"]
    assert st.rows == 33  # not 66: the up_proj call repeats the gate_proj input
    for e in range(4):
        assert torch.equal(st.expert_rows(e), _recorded(rec, "gate_proj", e, 32))
        assert torch.equal(st.expert_rows(e), _recorded(rec, "up_proj", e, 32))
        assert torch.equal(cap.stashes["down_proj"].expert_rows(e), _recorded(rec, "down_proj", e, 16))


def test_empty_batch_routes_nothing():
    st = capture.RoutedStash("s", 8, 3)
    st.add_routed(torch.zeros(0, 8), torch.zeros(0, 2, dtype=torch.int64))
    st.add_routed(torch.zeros(1, 0, 8), torch.zeros(0, 2, dtype=torch.int64))
    assert st.rows == 0 and st.token_counts().tolist() == [0, 0, 0]
    st.add_rows(1, torch.zeros(0, 8))
    st.add_routed(torch.ones(2, 8), torch.tensor([[0, 2], [2, 2]]))
    assert st.token_counts().tolist() == [1, 0, 3]
    blk = _block(E=4, k=2, hidden=32, inter=32)
    cap = capture.ExpertCapture(blk)
    with torch.no_grad(), cap:
        blk(torch.zeros(1, 0, 32))  # an empty batch through the real block
        blk(torch.randn(1, 5, 32))
    assert cap.stashes["experts.gate_up_proj"].rows == 5


def test_drop_expert_forgets_only_that_expert():
    st = capture.RoutedStash("s", 4, 3)
    x = torch.arange(12, dtype=torch.float32).reshape(3, 4)
    st.add_routed(x, torch.tensor([[0, 1], [1, 2], [2, 0]]))
    assert st.token_counts().tolist() == [2, 2, 2]
    st.drop_expert(1)
    assert st.token_counts().tolist() == [2, 0, 2]
    st.add_rows(1, torch.ones(1, 4))  # rows added after the drop count
    assert st.token_counts().tolist() == [2, 1, 2]
    assert torch.equal(st.expert_rows(1), torch.ones(1, 4, dtype=torch.bfloat16))
    assert sorted(st.expert_rows(0)[:, 0].tolist()) == [0.0, 8.0]


def test_clearing_one_sibling_view_keeps_the_other():
    """Separate gate_proj / up_proj parameters share one RoutedStash; the
    reference keeps one Stash per parameter and expert, and its clear() only
    empties that one (capture.py:78-79, .tokens kept). Clearing gate's view
    of expert e must leave up's rows of expert e in place."""
    st = capture.RoutedStash("s", 4, 3)
    x = torch.arange(12, dtype=torch.float32).reshape(3, 4)
    st.add_routed(x, torch.tensor([[0, 1], [1, 2], [2, 0]]))
    gate = capture.ExpertRows(st, 1, "m.gate_proj::e1")
    up = capture.ExpertRows(st, 1, "m.up_proj::e1")
    gate.clear()
    assert gate.tokens == 2 and gate.chunks == [] and gate.nbytes() == 0
    assert up.tokens == 2 and up.nbytes() == 2 * 4 * 2
    assert sorted(up.chunks[0][:, 0].tolist()) == [0.0, 4.0]
    assert st.token_counts().tolist() == [2, 2, 2]
    up.clear()  # the last view of expert 1: its rows go
    assert st.token_counts().tolist() == [2, 0, 2]
    assert up.tokens == 2 and gate.tokens == 2  # .tokens kept, as the reference's
    gate.clear()  # a second clear changes nothing
    assert gate.tokens == 2
