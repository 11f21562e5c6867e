"""Calibration-row stash and Hessian accumulation on MI355X.

``Stash`` keeps the reference's interface (mlx_gptq/capture.py:33-79: add,
add_sampled, nbytes, hessian, clear) and its numerics: captured rows are
rounded to bf16 (capture.py:49) and H = sum of x^T x in fp32. The product
differs in where rows live -- they stay on the device they were captured on
(HBM is large enough for a layer's calibration set) -- and in how H is
formed: one bf16-MFMA SYRK launch (csrc/hessian.hip) instead of chunked fp32
``addmm``.

``grouped_hessian`` is the batched form used for routed experts: every
expert's H from one hidden-state matrix plus a per-expert token list, with
the gather fused into the MFMA tile loads.

``RoutedStash`` and ``ExpertCapture`` are the routed-capture side of it
(the reference keeps one CPU ``Stash`` per expert, filled by intercepting
``F.linear`` on each expert's weight slice, capture.py:101-207): a fused
MoE expert module's input is stashed once per batch together with the
router's top-k assignment, so an expert's rows are never copied out; rows
that exist only per expert (the ``down_proj`` inputs) are appended with
their expert id. Every expert's H then comes from one grouped launch.
"""

from __future__ import annotations

import ctypes
import logging
import threading
from collections import OrderedDict
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np
import torch
import torch.nn.functional as F
from torch.overrides import TorchFunctionMode

from . import _native as nat

log = logging.getLogger(__name__)

# 3D expert parameter names of the transformers fused-expert layout
# (capture.py:28); the first three take the MoE block's hidden states.
FUSED_EXPERT_PARAMS = ("gate_up_proj", "gate_proj", "up_proj", "down_proj")
_INPUT_PARAMS = ("gate_up_proj", "gate_proj", "up_proj")


def _hip_device(device) -> torch.device:
    """`device` as an indexed HIP device; Hessians are formed on HIP devices
    only (there is no CPU path)."""
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError(
            "mlx_gptq (MI355X build) accumulates Hessians on HIP devices only "
            f"(got device {dev})"
        )
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


def _as_offsets(offsets) -> np.ndarray:
    if isinstance(offsets, torch.Tensor):
        offsets = offsets.detach().to("cpu", torch.int64).numpy()
    off = np.ascontiguousarray(np.asarray(offsets, dtype=np.int64))
    if off.ndim != 1 or off.size < 2:
        raise ValueError("offsets must be a 1-D sequence of n_groups + 1 entries")
    if np.any(np.diff(off) < 0) or off[0] < 0:
        raise ValueError("offsets must be non-negative and non-decreasing")
    return off


# Plans and device workspaces of recent grouped Hessian launches, keyed by
# (device, stream, C, offsets, target_items). A repeated launch (the same
# stash shape, layer after layer) skips the host planning, the pinned plan
# buffer, the workspace allocation and the plan's copy to the device. Launches
# on one stream run in order, so a cached workspace never serves two launches
# at once; other streams get their own entries.
_WS_CACHE: "OrderedDict[tuple, tuple[torch.Tensor, torch.Tensor]]" = OrderedDict()
_WS_CACHE_MAX_ENTRIES = 8
_WS_CACHE_MAX_BYTES = 512 << 20
_ws_lock = threading.Lock()


def _hessian_plan(dev: torch.device, stream: int, C: int, off: np.ndarray, target_items: int):
    """(plan, workspace): the pinned host plan and a device workspace that
    starts with a copy of it."""
    key = (dev.index, int(stream), C, off.tobytes(), int(target_items))
    with _ws_lock:
        hit = _WS_CACHE.get(key)
        if hit is not None:
            _WS_CACHE.move_to_end(key)
            return hit
    lib = nat.load()
    G = off.size - 1
    plan_bytes = ctypes.c_int64(0)
    ws_bytes = ctypes.c_int64(0)
    nat.check(
        lib.mgq_hessian_plan(C, G, off.ctypes.data, int(target_items), None, 0,
                             ctypes.byref(plan_bytes), ctypes.byref(ws_bytes)),
        "mgq_hessian_plan",
    )
    plan = torch.empty(plan_bytes.value, dtype=torch.uint8, pin_memory=True)
    nat.check(
        lib.mgq_hessian_plan(C, G, off.ctypes.data, int(target_items), plan.data_ptr(),
                             plan_bytes.value, None, None),
        "mgq_hessian_plan",
    )
    ws = torch.empty(ws_bytes.value, dtype=torch.uint8, device=dev)
    ws[: plan_bytes.value].copy_(plan, non_blocking=True)
    with _ws_lock:
        _WS_CACHE[key] = (plan, ws)
        total = sum(w.numel() for _, w in _WS_CACHE.values())
        while _WS_CACHE and (len(_WS_CACHE) > _WS_CACHE_MAX_ENTRIES or total > _WS_CACHE_MAX_BYTES):
            _, (_, w) = _WS_CACHE.popitem(last=False)
            total -= w.numel()
    return plan, ws


def clear_hessian_plan_cache() -> None:
    """Forget every cached Hessian launch plan and its device workspace.
    The next launch of each shape plans again, as the first launch for a new
    routing (a new layer's offsets) does; the workspaces go back to torch's
    allocator."""
    with _ws_lock:
        _WS_CACHE.clear()


def grouped_hessian(
    X: torch.Tensor,
    offsets: Sequence[int] | np.ndarray | torch.Tensor,
    row_index: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
    target_items: int = 0,
    validate: bool = True,
) -> torch.Tensor:
    """H[g] (+)= X_g^T X_g for every group g, fp32 [G, C, C].

    X: bf16 [N, C] on a HIP device (row-contiguous; any C, a C that is not a
    multiple of 8 or rows that are not 16-byte aligned go through a padded
    copy). Group g uses the token
    list entries offsets[g]:offsets[g+1]; entry t selects row
    ``row_index[t]`` of X (or row t when ``row_index`` is None).
    ``validate`` checks the gather indices first (one device reduction and a
    host sync); the kernel never reads outside X either way.
    """
    if X.dtype != torch.bfloat16:
        raise TypeError(f"grouped_hessian expects bfloat16 rows (got {X.dtype})")
    if X.dim() != 2 or X.stride(1) != 1:
        raise ValueError("X must be a row-contiguous [N, C] matrix")
    dev = nat.device_for(X)
    if not X.is_cuda:
        X = X.to(dev)
    off = _as_offsets(offsets)
    G = off.size - 1
    C = int(X.shape[1])
    if row_index is not None:
        row_index = nat.on_device(row_index.to(torch.int32), dev)
        if int(off[-1]) > row_index.numel():
            raise ValueError("offsets exceed the token list")
        if validate and row_index.numel():
            lo, hi = torch.aminmax(row_index[: int(off[-1])])
            if int(lo) < 0 or int(hi) >= X.shape[0]:
                raise IndexError(f"row_index outside [0, {X.shape[0]})")
    elif int(off[-1]) > X.shape[0]:
        raise ValueError("offsets exceed the rows of X")
    if out is not None and (out.shape != (G, C, C) or out.dtype != torch.float32
                            or not out.is_contiguous()):
        raise ValueError(f"out must be a contiguous float32 [{G}, {C}, {C}] tensor")
    if C % 8 or X.stride(0) % 8 or X.data_ptr() % 16:
        # The kernel moves rows in 16-byte pieces. Zero columns add nothing
        # to X^T X, so such X is solved as a zero-padded copy and H is the
        # padded result's leading C x C block.
        C8 = -(-C // 8) * 8
        Xp = torch.zeros(X.shape[0], C8, dtype=torch.bfloat16, device=dev)
        Xp[:, :C] = X
        Hp = grouped_hessian(Xp, off, row_index, None, False, target_items, validate=False)
        if out is None:
            return Hp[:, :C, :C].contiguous()
        if accumulate:
            out += Hp[:, :C, :C]
        else:
            out.copy_(Hp[:, :C, :C])
        return out
    if out is None:
        out = torch.empty(G, C, C, dtype=torch.float32, device=dev)
        accumulate = False
    stream = nat.stream_of(dev)
    plan, ws = _hessian_plan(dev, stream, C, off, target_items)
    nat.call(
        "mgq_hessian", X.data_ptr(), int(X.shape[0]), X.stride(0), C,
        None if row_index is None else row_index.data_ptr(), plan.data_ptr(), out.data_ptr(),
        1 if accumulate else 0, ws.data_ptr(), ws.numel(), stream,
    )
    return out


def hessian_xtx(X: torch.Tensor, out: torch.Tensor | None = None, accumulate: bool = False) -> torch.Tensor:
    """Dense H = X^T X (fp32 [C, C]) of bf16 rows X [N, C]."""
    H = grouped_hessian(X, [0, int(X.shape[0])], None,
                        None if out is None else out.unsqueeze(0), accumulate)
    return H[0]


class Stash:
    """Captured input rows for one logical weight matrix (capture.py:33-79)."""

    def __init__(self, name: str, in_features: int):
        self.name = name
        self.in_features = in_features
        self.chunks: list[torch.Tensor] = []
        self.tokens = 0

    def add(self, x: torch.Tensor):
        rows = x.detach().reshape(-1, x.shape[-1])
        if rows.shape[-1] != self.in_features:
            raise RuntimeError(
                f"stash {self.name}: got rows of dim {rows.shape[-1]}, "
                f"expected {self.in_features}"
            )
        # bf16 rounding as capture.py:49; rows stay on their device, in a
        # copy of their own (the caller may reuse its input buffer).
        self.chunks.append(rows.to(torch.bfloat16, copy=True).contiguous())
        self.tokens += rows.shape[0]

    def add_sampled(self, x: torch.Tensor, max_rows: int):
        """Deterministic, evenly spaced sample of rows (capture.py:52-63)."""
        rows = x.detach().reshape(-1, x.shape[-1])
        if rows.shape[0] > max_rows:
            idx = torch.linspace(0, rows.shape[0] - 1, steps=max_rows, device=rows.device).long()
            rows = rows.index_select(0, idx)
        self.add(rows)

    def nbytes(self) -> int:
        return sum(c.numel() * 2 for c in self.chunks)

    def rows_on(self, device) -> torch.Tensor:
        """Every stored row as one contiguous bf16 [tokens, C] matrix on
        `device`. The chunks are joined (and moved) once; the joined matrix
        then replaces them, so later calls cost nothing."""
        dev = torch.device(device)
        if not self.chunks:
            return torch.zeros(0, self.in_features, dtype=torch.bfloat16, device=dev)
        if len(self.chunks) == 1 and self.chunks[0].device == dev:
            return self.chunks[0]
        X = torch.cat([c.to(dev, non_blocking=True) for c in self.chunks])
        self.chunks = [X]
        return X

    @torch.no_grad()
    def hessian(self, device, chunk_rows: int = 65536) -> torch.Tensor:
        """H = X^T X in fp32 on `device` (capture.py:68-76).

        One SYRK launch over all stored rows: the kernel splits the token
        range across workgroups itself, so there is no per-chunk launch or
        read-modify-write of H. ``chunk_rows`` is accepted for signature
        compatibility; in the reference it only sets the fp32 summation
        blocks of its ``addmm`` loop."""
        dev = _hip_device(device)
        X = self.rows_on(dev)
        if X.shape[0] == 0:
            return torch.zeros(self.in_features, self.in_features, dtype=torch.float32, device=dev)
        return hessian_xtx(X)

    def clear(self):
        self.chunks.clear()


class RoutedStash:
    """Calibration rows of every expert of one fused [E, out, in] parameter.

    Holds what the reference keeps as E per-expert stashes (keys
    ``{module}.{param}::e{e}``, capture.py:149-153, each filled with the rows
    routed to that expert, capture.py:192-207) as one append-only bf16 row
    buffer on the capture device plus an (expert, row) assignment list:

    * ``add_routed(x, top_k_index)``: the block's input rows, stored once,
      and the router's choice for each (expert ids outside [0, E) are
      dropped, as the eager expert loop skips them);
    * ``add_rows(expert, x)``: rows that exist for one expert only (the
      ``down_proj`` inputs).

    ``hessians`` forms H_e = X_e^T X_e (fp32) for a span of experts in one
    grouped SYRK launch, gathering each expert's rows inside the kernel.
    Rows are rounded to bf16 as capture.py:49 does; the row order inside
    an expert differs from the eager loop's, which changes only the fp32
    summation order of H.

    ``expert_hessian`` serves the reference's one-expert-at-a-time
    ``stashes[key].hessian(device)`` calls (sequential.py:546-551): the
    first call for expert e forms the Hessians of a whole span e, e+1, ...
    (up to ``span_bytes`` of them) in one launch and hands the rest out
    from a cache on the following calls.
    """

    def __init__(self, name: str, in_features: int, num_experts: int,
                 span_bytes: int = 1 << 30):
        self.name = name
        self.in_features = int(in_features)
        self.num_experts = int(num_experts)
        self.span_bytes = int(span_bytes)
        self.chunks: list[torch.Tensor] = []
        self._experts: list[torch.Tensor] = []  # int32 expert id per assignment
        self._rows: list[torch.Tensor] = []  # int32 row of the buffer per assignment
        self._pending: list[tuple[int, torch.Tensor]] = []  # (first row, top-k ids [T, k])
        self.rows = 0  # rows stored
        self._plan = None
        self._hcache: dict[tuple[int, torch.device], torch.Tensor] = {}
        # per expert: the names of the ExpertRows views over it, and those of
        # them that were cleared; rows are dropped once every view is
        self._views: dict[int, set[str]] = {}
        self._released: dict[int, set[str]] = {}
        self._lock = threading.RLock()

    def _append(self, x: torch.Tensor) -> tuple[torch.Tensor, int]:
        rows = x.detach().reshape(-1, x.shape[-1])
        if rows.shape[-1] != self.in_features:
            raise RuntimeError(
                f"stash {self.name}: got rows of dim {rows.shape[-1]}, "
                f"expected {self.in_features}"
            )
        base = self.rows
        if base + rows.shape[0] > 2**31 - 1:
            raise RuntimeError(f"stash {self.name}: more than 2^31 - 1 rows")
        if rows.shape[0]:
            self.chunks.append(rows.to(torch.bfloat16, copy=True).contiguous())
            self.rows += rows.shape[0]
            self._plan = None
            self._hcache.clear()
        return rows, base

    def add_routed(self, x: torch.Tensor, top_k_index: torch.Tensor):
        """Rows x [T, C] (any leading shape) routed to experts
        top_k_index [T, k] (the router's top-k choice per row)."""
        rows, base = self._append(x)
        T = rows.shape[0]
        ti = top_k_index.detach()
        if ti.dtype.is_floating_point or ti.numel() % max(T, 1) != 0:
            raise ValueError(f"stash {self.name}: top_k_index must hold k integer ids per row")
        if T == 0:
            return  # an empty batch routes nothing
        # the (expert, row) lists are built by plan(), for all batches at once
        self._pending.append((base, ti.reshape(T, -1).to(device=rows.device, copy=True)))

    def _assign(self, ti: torch.Tensor, base: int):
        T, k = ti.shape
        e = ti.reshape(-1).to(torch.int64)
        e = torch.where((e >= 0) & (e < self.num_experts), e, self.num_experts).to(torch.int32)
        r = (torch.arange(T, device=ti.device, dtype=torch.int32) + base).repeat_interleave(k)
        self._experts.append(e)
        self._rows.append(r)

    def _materialize(self):
        p = self._pending
        if not p:
            return
        same_k = len({ti.shape[1] for _, ti in p}) == 1
        back_to_back = all(p[i + 1][0] == p[i][0] + p[i][1].shape[0] for i in range(len(p) - 1))
        if same_k and back_to_back:
            self._assign(p[0][1] if len(p) == 1 else torch.cat([ti for _, ti in p]), p[0][0])
        else:
            for base, ti in p:
                self._assign(ti, base)
        self._pending = []

    def add_rows(self, expert: int, x: torch.Tensor):
        """Rows x that belong to `expert` alone."""
        if not 0 <= int(expert) < self.num_experts:
            raise IndexError(f"stash {self.name}: expert {expert} outside [0, {self.num_experts})")
        rows, base = self._append(x)
        n = rows.shape[0]
        if n == 0:
            return
        self._experts.append(torch.full((n,), int(expert), dtype=torch.int32, device=rows.device))
        self._rows.append(torch.arange(base, base + n, dtype=torch.int32, device=rows.device))

    def nbytes(self) -> int:
        return (sum(c.numel() * 2 for c in self.chunks) + sum(r.numel() * 8 for r in self._rows)
                + sum(ti.numel() * ti.element_size() for _, ti in self._pending))

    def plan(self) -> tuple[torch.Tensor, np.ndarray, torch.Tensor]:
        """(X, offsets, row_index): X bf16 [rows, C], the stored rows;
        expert e's rows are X[row_index[offsets[e]:offsets[e + 1]]]
        (offsets int64 [E + 1] on the host, row_index int32 on X's device).
        One host sync (the per-expert counts)."""
        if self._plan is None:
            if not self.chunks:
                raise RuntimeError(f"stash {self.name}: nothing captured")
            X = self.chunks[0] if len(self.chunks) == 1 else torch.cat(self.chunks)
            self.chunks = [X]
            self._materialize()
            if not self._experts:
                raise RuntimeError(f"stash {self.name}: nothing captured")
            e = torch.cat(self._experts)
            r = torch.cat(self._rows)
            e_sorted, order = torch.sort(e, stable=True)
            row_index = r[order].contiguous()
            counts = torch.bincount(e_sorted, minlength=self.num_experts + 1)[: self.num_experts]
            off = np.zeros(self.num_experts + 1, dtype=np.int64)
            off[1:] = np.cumsum(counts.cpu().numpy())
            self._experts, self._rows = [e_sorted], [row_index]
            self._plan = (X, off, row_index)
        return self._plan

    def token_counts(self) -> np.ndarray:
        """Rows per expert (int64 [E])."""
        if not self.chunks:
            return np.zeros(self.num_experts, dtype=np.int64)
        return np.diff(self.plan()[1])

    def expert_rows(self, expert: int) -> torch.Tensor:
        """Expert `expert`'s rows, gathered (bf16 [n, C])."""
        X, off, ri = self.plan()
        return X.index_select(0, ri[int(off[expert]) : int(off[expert + 1])].long())

    @torch.no_grad()
    def hessians(self, device=None, experts: range | None = None,
                 out: torch.Tensor | None = None) -> torch.Tensor:
        """H_e = X_e^T X_e, fp32 [len(experts), C, C], for experts
        e0..e1-1 (default: all), as sequential.py:546-551 stacks per-expert
        Stash.hessian results; experts without rows get H = 0."""
        E = self.num_experts
        experts = range(E) if experts is None else experts
        if experts.step != 1 or not 0 <= experts.start <= experts.stop <= E:
            raise ValueError(f"experts must be a contiguous span inside [0, {E})")
        C = self.in_features
        with self._lock:
            if not self.chunks:
                dev = _hip_device("cuda" if device is None else device)
                H = torch.zeros(len(experts), C, C, dtype=torch.float32, device=dev)
                if out is not None:
                    out.copy_(H)
                    return out
                return H
            X, off, ri = self.plan()
            if device is not None:
                dev = _hip_device(device)
                if X.device != dev:
                    X, ri = X.to(dev), ri.to(dev)
                    self.chunks, self._rows = [X], [ri]
                    self._plan = (X, off, ri)
        return grouped_hessian(X, off[experts.start : experts.stop + 1], ri, out=out,
                               validate=False)

    def expert_hessian(self, expert: int, device=None) -> torch.Tensor:
        """One expert's H (fp32 [C, C]) for a caller that asks expert by
        expert. A miss forms the Hessians of experts expert..expert+n-1
        (n such that they fit in ``span_bytes``) in one grouped launch and
        keeps the others for the following calls; each cached H is handed
        out once."""
        e = int(expert)
        if not 0 <= e < self.num_experts:
            raise IndexError(f"stash {self.name}: expert {e} outside [0, {self.num_experts})")
        with self._lock:
            dev = _hip_device("cuda" if device is None else device)
            H = self._hcache.pop((e, dev), None)
            if H is not None:
                return H
            C = self.in_features
            n = max(1, min(self.num_experts - e, self.span_bytes // max(C * C * 4, 1)))
            Hs = self.hessians(dev, range(e, e + n))
            for i in range(1, n):
                self._hcache[(e + i, dev)] = Hs[i]
            return Hs[0]

    def hessian(self, expert: int, device=None) -> torch.Tensor:
        """One expert's H (fp32 [C, C]), the per-expert Stash.hessian."""
        return self.hessians(device, range(int(expert), int(expert) + 1))[0]

    def drop_expert(self, expert: int):
        """Forget expert `expert`'s rows (the per-expert Stash.clear)."""
        e = int(expert)
        with self._lock:
            self._materialize()
            for ids in self._experts:  # its assignments go to the ignored id E
                ids.masked_fill_(ids == e, self.num_experts)
            self._plan = None
            self._hcache.clear()

    def attach_view(self, expert: int, name: str):
        """Register a per-expert view (``ExpertRows``) of expert `expert`."""
        with self._lock:
            self._views.setdefault(int(expert), set()).add(name)
            self._released.get(int(expert), set()).discard(name)

    def release_view(self, expert: int, name: str):
        """View `name` of expert `expert` was cleared. Separate gate_proj /
        up_proj parameters share this stash, while the reference keeps one
        Stash per parameter and expert: the rows are dropped only once every
        view of the expert has been cleared, so clearing one sibling leaves
        the other's rows in place."""
        e = int(expert)
        with self._lock:
            rel = self._released.setdefault(e, set())
            rel.add(name)
            if rel >= self._views.get(e, set()):
                self.drop_expert(e)

    def clear(self):
        with self._lock:
            self.chunks.clear()
            self._experts.clear()
            self._rows.clear()
            self._pending.clear()
            self.rows = 0
            self._plan = None
            self._hcache.clear()
            self._released.clear()


class ExpertCapture:
    """Routed capture of every fused MoE expert parameter under `root`.

    Finds the modules that own 3D ``gate_up_proj`` / ``gate_proj`` /
    ``up_proj`` / ``down_proj`` parameters [E, out, in] (the detection of
    capture.py:133-158) and gives each parameter a ``RoutedStash``
    (``stashes["{module}.{param}"]``; the input parameters of one module
    share one). While active:

    * a forward pre-hook on each such module stashes its input
      (``hidden_states``) once, with the ``top_k_index`` it is called with
      (the transformers expert-module signature ``forward(hidden_states,
      top_k_index, top_k_weights)``);
    * a TorchFunctionMode matches ``F.linear`` weights against each expert
      slice's data pointer, as capture.py:192-207 does, and appends the
      ``down_proj`` inputs to expert e's rows. For a module called without
      a usable ``top_k_index`` the input parameters are captured the same
      way (rows copied per expert, still on device).
    """

    def __init__(self, root: torch.nn.Module, group_size: int | None = None):
        self.stashes: dict[str, RoutedStash] = {}
        self.params: dict[str, tuple[str, str, torch.nn.Parameter]] = {}
        self._modules: dict[str, torch.nn.Module] = {}
        self._input_key: dict[str, str] = {}  # module name -> shared input stash key
        self._ptr: dict[int, tuple[str, int, str]] = {}  # slice ptr -> (key, expert, module)
        self._routed: dict[str, bool] = {}
        self._samples: dict[str, Stash] = {}  # module -> sampled block inputs (backfill source)
        # module -> {expert: the input tensor last stored for it in the current
        # call}: separate gate_proj / up_proj slices see the same tensor and
        # share one stash, so the second F.linear must not store it again
        self._last_in: dict[str, dict[int, torch.Tensor]] = {}
        self.fallback_experts: dict[str, str] = {}
        self._hooks = []
        self._mode = None
        self.skipped: list[str] = []
        for name, mod in root.named_modules():
            for pname, p in mod.named_parameters(recurse=False):
                if p.dim() != 3 or pname not in FUSED_EXPERT_PARAMS:
                    continue
                key = f"{name}.{pname}" if name else pname
                E, C = p.shape[0], p.shape[-1]
                if group_size and C % group_size != 0:
                    log.warning("skipping fused %s.%s: in dim %d not divisible by group %d",
                                name, pname, C, group_size)
                    self.skipped.append(key)
                    continue
                if pname in _INPUT_PARAMS:
                    ik = self._input_key.setdefault(name, key)
                    if ik not in self.stashes:
                        self.stashes[ik] = RoutedStash(f"{name}::inputs", C, E)
                        self._samples[name] = Stash(f"{name}::all_inputs", C)
                    self.stashes[key] = self.stashes[ik]
                else:
                    self.stashes[key] = RoutedStash(key, C, E)
                self.params[key] = (name, pname, p)
                self._modules[name] = mod
                for e in range(E):
                    ptr = p.data_ptr() + e * p.stride(0) * p.element_size()
                    self._ptr[ptr] = (key, e, name)

    # ---- hooks ----------------------------------------------------------

    def _make_pre_hook(self, name: str):
        def hook(mod, args, kwargs):
            x = args[0] if args else kwargs.get("hidden_states")
            ti = args[1] if len(args) > 1 else kwargs.get("top_k_index")
            ik = self._input_key.get(name)
            ok = (
                ik is not None
                and isinstance(x, torch.Tensor)
                and isinstance(ti, torch.Tensor)
                and not ti.dtype.is_floating_point
                and ti.dim() >= 1
                and x.dim() >= 1
                and ti.numel() % max(x.numel() // x.shape[-1], 1) == 0
            )
            self._routed[name] = bool(ok)
            self._last_in[name] = {}
            if ok:
                self.stashes[ik].add_routed(x, ti)
            if ik is not None and isinstance(x, torch.Tensor):
                # 64 evenly spaced rows per batch: the activation-aware
                # fallback for experts the router never picks (capture.py:177-184)
                self._samples[name].add_sampled(x, 64)
        return hook

    class _Mode(TorchFunctionMode):
        def __init__(self, cap):
            super().__init__()
            self.cap = cap

        def __torch_function__(self, func, types, args=(), kwargs=None):
            kwargs = kwargs or {}
            if func is F.linear and len(args) >= 2:
                w = args[1]
                if isinstance(w, torch.Tensor) and w.dim() == 2:
                    hit = self.cap._ptr.get(w.data_ptr())
                    if hit is not None:
                        key, e, name = hit
                        st = self.cap.stashes[key]
                        if w.shape[-1] == st.in_features and self.cap._take(key, e, name, args[0]):
                            st.add_rows(e, args[0])
            return func(*args, **kwargs)

    def _take(self, key: str, e: int, name: str, x) -> bool:
        """Whether an expert slice's F.linear input is stored: always for
        ``down_proj``; for the input parameters only when the module call
        was not routed through the pre-hook, and only once per tensor and
        expert in one call."""
        if self.params[key][1] not in _INPUT_PARAMS:
            return True
        if self._routed.get(name):
            return False
        seen = self._last_in.setdefault(name, {})
        if seen.get(e) is x:
            return False
        seen[e] = x
        return True

    def __enter__(self):
        for name, mod in self._modules.items():
            self._hooks.append(mod.register_forward_pre_hook(self._make_pre_hook(name), with_kwargs=True))
        if self._ptr:
            self._mode = self._Mode(self)
            self._mode.__enter__()
        return self

    def __exit__(self, *exc):
        if self._mode is not None:
            self._mode.__exit__(*exc)
            self._mode = None
        for h in self._hooks:
            h.remove()
        self._hooks.clear()
        self._last_in.clear()
        return False

    # ---- results ----------------------------------------------------------

    def hessians(self, key: str, device=None, experts: range | None = None) -> torch.Tensor:
        """Stacked expert Hessians of parameter `key` (see RoutedStash.hessians)."""
        return self.stashes[key].hessians(device, experts)

    def expert_token_stats(self) -> dict[str, tuple[int, int, int, int]]:
        """key -> (min, median, max, zero_count) of rows per expert
        (capture.py:238-248)."""
        out = {}
        for key in self.params:
            c = np.sort(self.stashes[key].token_counts())
            out[key] = (int(c[0]), int(c[len(c) // 2]), int(c[-1]), int((c == 0).sum()))
        return out

    def check_capture_happened(self):
        """Abort when a fused parameter got no rows at all (capture.py:320-330)."""
        for key in self.params:
            if self.stashes[key].rows == 0:
                raise RuntimeError(
                    f"No tokens captured for fused experts {key}. The expert loop did not "
                    "call the module with top_k_index nor F.linear on the expert slices; "
                    "load the model with experts_implementation='eager'."
                )

    @torch.no_grad()
    def backfill_unrouted_experts(self) -> dict[str, list[int]]:
        """Rows for experts that got none (capture.py:250-318): the block's
        sampled inputs for the input parameters, and for ``down_proj`` the
        activations SiLU(gate) * up of those rows under that expert's own
        weights. Returns module -> backfilled experts; the affected
        ``{key}::e{e}`` names are listed in ``fallback_experts``."""
        out: dict[str, list[int]] = {}
        for name, ik in self._input_key.items():
            src = self._samples.get(name)
            if src is None or src.tokens == 0:
                continue
            st = self.stashes[ik]
            counts = st.token_counts()
            missing = [e for e in range(st.num_experts) if counts[e] == 0]
            if not missing:
                continue
            params = {pn: p for (mn, pn, p) in self.params.values() if mn == name}
            in_keys = [k for k, (mn, pn, _) in self.params.items() if mn == name and pn in _INPUT_PARAMS]
            dk = next((k for k, (mn, pn, _) in self.params.items() if mn == name and pn == "down_proj"), None)
            for e in missing:
                for chunk in src.chunks:
                    st.add_rows(e, chunk)
                for k in in_keys:
                    self.fallback_experts[f"{k}::e{e}"] = "all_expert_inputs"
                if dk is None:
                    continue
                down = self.stashes[dk]
                before = down.rows
                for chunk in src.chunks:
                    if "gate_up_proj" in params:
                        w = params["gate_up_proj"][e]
                        gate, up = F.linear(chunk.to(w.device, w.dtype), w).chunk(2, dim=-1)
                        down.add_rows(e, F.silu(gate) * up)
                    elif "gate_proj" in params and "up_proj" in params:
                        wg, wu = params["gate_proj"][e], params["up_proj"][e]
                        x = chunk.to(wg.device, wg.dtype)
                        down.add_rows(e, F.silu(F.linear(x, wg)) * F.linear(x, wu))
                if down.rows > before:
                    self.fallback_experts[f"{dk}::e{e}"] = "all_expert_inputs"
            out[name] = missing
        return out

    def drop_all(self):
        for st in self.stashes.values():
            st.clear()
        for st in self._samples.values():
            st.clear()


# --------------------------------------------------------------------------
# The reference's capture interface for one decoder layer (capture.py:82-343)
# --------------------------------------------------------------------------


@dataclass
class LinearTask:
    """An ``nn.Linear`` of the layer to quantize (capture.py:82-87).
    ``stash_key`` names the stash holding its input rows; the same-input
    dedup re-points it at a sibling's stash."""

    name: str
    module: torch.nn.Module
    stash_key: str


@dataclass
class FusedExpertTask:
    """One fused 3D expert parameter [E, out, in], quantized per expert
    (capture.py:90-97). ``stash_keys[e]`` is ``"{module_name}.{param_name}::e{e}"``."""

    module_name: str
    param_name: str
    param: torch.nn.Parameter
    num_experts: int
    stash_keys: list[str] = field(default_factory=list)


class ExpertRows:
    """Expert `expert`'s rows of a ``RoutedStash``, behind the per-expert
    ``Stash`` interface the reference's callers use (``hessian``,
    ``tokens``, ``chunks``, ``add``, ``nbytes``, ``clear``). No rows are
    copied out: ``hessian`` is served from the stash's grouped launch."""

    def __init__(self, routed: RoutedStash, expert: int, name: str):
        self.routed = routed
        self.expert = int(expert)
        self.name = name
        self.in_features = routed.in_features
        # set by clear(): the token count kept, as the reference's Stash.clear
        # keeps .tokens (capture.py:78-79) while its rows are gone
        self._kept_tokens: int | None = None
        routed.attach_view(self.expert, name)

    @property
    def tokens(self) -> int:
        if self._kept_tokens is not None:
            return self._kept_tokens
        return int(self.routed.token_counts()[self.expert])

    @property
    def chunks(self) -> list[torch.Tensor]:
        """This expert's rows, gathered into one bf16 [tokens, C] matrix."""
        if self._kept_tokens is not None or self.tokens == 0:
            return []
        return [self.routed.expert_rows(self.expert)]

    def add(self, x: torch.Tensor):
        # rows added after a clear make the view live again over the shared
        # stash (a sibling that was not cleared keeps its earlier rows there)
        if self._kept_tokens is not None:
            self._kept_tokens = None
            self.routed.attach_view(self.expert, self.name)
        self.routed.add_rows(self.expert, x)

    def add_sampled(self, x: torch.Tensor, max_rows: int):
        rows = x.detach().reshape(-1, x.shape[-1])
        if rows.shape[0] > max_rows:
            idx = torch.linspace(0, rows.shape[0] - 1, steps=max_rows, device=rows.device).long()
            rows = rows.index_select(0, idx)
        self.add(rows)

    def nbytes(self) -> int:
        if self._kept_tokens is not None:
            return 0
        return self.tokens * self.in_features * 2

    @torch.no_grad()
    def hessian(self, device, chunk_rows: int = 65536) -> torch.Tensor:
        """H = X_e^T X_e in fp32 on `device` (capture.py:68-76); zeros once
        this view was cleared, as the reference's emptied Stash gives."""
        dev = _hip_device(device)
        if self._kept_tokens is not None:
            return torch.zeros(self.in_features, self.in_features, dtype=torch.float32, device=dev)
        return self.routed.expert_hessian(self.expert, dev)

    def clear(self):
        if self._kept_tokens is None:
            self._kept_tokens = self.tokens
            self.routed.release_view(self.expert, self.name)


class CaptureManager:
    """All capture state and hooks of one decoder layer (capture.py:100-343).

    Same constructor, attributes and methods as the reference, so the
    Stage-A drivers (sequential.py:707-741, dflash2_calibrate.py:177-214)
    run on it unchanged; rows stay in HBM instead of CPU bf16 stashes:

    * ``nn.Linear`` modules (not matching ``exclude_regex``, in_features
      divisible by ``group_size``) become ``LinearTask``s with a
      ``Stash`` each; a forward pre-hook stores the module's input, once per
      batch per input tensor -- q/k/v or gate/up called on the same tensor
      share the first sibling's stash (the task's ``stash_key`` is
      re-pointed, as the reference does).
    * fused 3D expert parameters become ``FusedExpertTask``s captured by an
      ``ExpertCapture`` (the block input stored once per batch with its
      top-k ids); ``stashes["{module}.{param}::e{e}"]`` are ``ExpertRows``
      views of it.

    Fast paths beyond the reference: ``expert_hessians(task, device,
    experts)`` for a span of experts in one launch, and
    ``span_solve.solve_fused_task`` for the whole task.
    """

    def __init__(self, layer: torch.nn.Module, exclude_regex, group_size: int):
        import re

        self.layer = layer
        self.group_size = int(group_size)
        self.stashes: dict[str, Stash | ExpertRows] = {}
        self.linear_tasks: list[LinearTask] = []
        self.fused_tasks: list[FusedExpertTask] = []
        self._hooks = []
        self._batch_seen: dict[int, tuple[torch.Tensor, str]] = {}
        excl = re.compile(exclude_regex) if exclude_regex else None
        for name, mod in layer.named_modules():
            if not isinstance(mod, torch.nn.Linear):
                continue
            if excl is not None and excl.search(name):
                log.debug("excluding %s (matches exclude regex)", name)
                continue
            if mod.in_features % self.group_size != 0:
                log.warning("skipping %s: in_features %d not divisible by group %d "
                            "(stays unquantized)", name, mod.in_features, self.group_size)
                continue
            self.linear_tasks.append(LinearTask(name, mod, stash_key=name))
            self.stashes.setdefault(name, Stash(name, mod.in_features))
        self.experts = ExpertCapture(layer, self.group_size)
        self._task_stash: dict[int, RoutedStash] = {}
        for key, (mname, pname, p) in self.experts.params.items():
            E = int(p.shape[0])
            task = FusedExpertTask(mname, pname, p, E)
            st = self.experts.stashes[key]
            for e in range(E):
                k = f"{mname}.{pname}::e{e}"
                task.stash_keys.append(k)
                self.stashes[k] = ExpertRows(st, e, k)
            self._task_stash[id(task)] = st
            self.fused_tasks.append(task)

    @property
    def fallback_experts(self) -> dict[str, str]:
        """stash key -> "all_expert_inputs" for backfilled experts."""
        out = {}
        for k, v in self.experts.fallback_experts.items():
            base, _, e = k.rpartition("::e")
            mname, pname, _ = self.experts.params[base]
            out[f"{mname}.{pname}::e{e}"] = v
        return out

    # ---- nn.Linear capture --------------------------------------------------

    def _linear_hook(self, task: LinearTask):
        def hook(mod, args, kwargs):
            x = args[0] if args else kwargs.get("input")
            seen = self._batch_seen.get(id(x))
            if seen is not None and seen[0] is x:
                task.stash_key = seen[1]  # a sibling already stored this tensor
                return
            self._batch_seen[id(x)] = (x, task.stash_key)
            self.stashes[task.stash_key].add(x)
        return hook

    # ---- lifecycle -------------------------------------------------------------

    def __enter__(self):
        for t in self.linear_tasks:
            self._hooks.append(t.module.register_forward_pre_hook(self._linear_hook(t),
                                                                  with_kwargs=True))
        self.experts.__enter__()
        return self

    def __exit__(self, *exc):
        self.experts.__exit__(*exc)
        for h in self._hooks:
            h.remove()
        self._hooks.clear()
        self._batch_seen.clear()
        return False

    def begin_batch(self):
        """A new calibration batch: input tensors seen so far no longer dedup."""
        self._batch_seen.clear()

    # ---- diagnostics and results ---------------------------------------------

    def total_stash_bytes(self) -> int:
        lin = sum(s.nbytes() for s in self.stashes.values() if isinstance(s, Stash))
        routed = {id(st): st for st in self.experts.stashes.values()}
        return lin + sum(st.nbytes() for st in routed.values())

    def expert_token_stats(self) -> dict[str, tuple[int, int, int, int]]:
        """"{module}.{param}" -> (min, median, max, zero_count) of tokens per
        expert (capture.py:242-252)."""
        out = {}
        for t in self.fused_tasks:
            c = np.sort(self._task_stash[id(t)].token_counts())
            out[f"{t.module_name}.{t.param_name}"] = (int(c[0]), int(c[len(c) // 2]), int(c[-1]),
                                                      int((c == 0).sum()))
        return out

    def backfill_unrouted_experts(self) -> dict[str, list[int]]:
        """Activation-aware rows for never-routed experts (capture.py:254-322);
        returns module name -> backfilled experts."""
        return self.experts.backfill_unrouted_experts()

    def check_capture_happened(self):
        """Abort if a fused parameter received no rows at all (capture.py:328-337)."""
        for t in self.fused_tasks:
            if self._task_stash[id(t)].rows == 0:
                raise RuntimeError(
                    f"No tokens captured for fused experts {t.module_name}.{t.param_name}. "
                    "The model is probably not using the eager experts implementation; "
                    "load it with experts_implementation='eager'."
                )

    def expert_hessians(self, task: FusedExpertTask, device, experts: range | None = None,
                        out: torch.Tensor | None = None) -> torch.Tensor:
        """Stacked H of a span of the task's experts (fp32 [n, C, C]), one launch."""
        return self._task_stash[id(task)].hessians(device, experts, out=out)

    def drop_all(self):
        for s in self.stashes.values():
            if isinstance(s, Stash):
                s.clear()
        self.experts.drop_all()
