"""Stacked-expert IQ_K module with the ``(x, indices, sorted_indices)`` switch interface.

The drop-in for the reference's ``IqkSwitchLinear`` (src/mlx_iqk/nn.py:105-333)
on PyTorch-ROCm: same constructor, same stream contract (the relayout
streams are module buffers named and shaped by the format), same call seam,
same route choice (src/mlx_iqk/nn.py:49, 221-238):

* **decode** (``indices.numel() <= DECODE_MAT_LIMIT`` and not sorted): the
  fused GEMV streams the selected experts' relayout directly;
* **prefill** (otherwise): by default the fused contraction forms each
  routed expert's fp16 weights -- the producer's values, bit for bit --
  inside an fp16 MFMA grouped GEMM and never stores them
  (``fused_prefill = True``); with ``fused_prefill = False`` the producer
  reconstructs each routed expert once into an fp16 stack and a sorted
  grouped GEMM contracts it.  The reference dequantizes every expert and
  calls ``mx.gather_mm``; here only the routed experts are touched, and the
  pair sort, grouping and un-permute happen on the device with no host
  synchronisation.

Shapes follow the reference: gate/up pass ``x [..., 1, 1, in]`` (one row per
token shared by its ``top_k`` experts), down passes ``x [..., top_k, 1, in]``
(one row per pair); ``indices`` is ``[..., top_k]``; the result is
``[..., top_k, 1, out]``.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import kernels
from .format import IQ2NL_VALUES, check_member, component_shapes
from .iq1grid import grid_values
from .kernels import IqkKernelError, check_dequant_geometry, check_gemv_geometry, stream_dtypes

DECODE_MAT_LIMIT = 63
"""Token-expert pairs at or below which the decode GEMV serves
(reference: src/mlx_iqk/nn.py:49-54)."""


class IqkRuntimeError(RuntimeError):
    pass


_TABLES: dict[tuple, torch.Tensor] = {}


def value_table(device=None) -> torch.Tensor:
    """The fp16 ``iq2nl_values`` table, one shared tensor per device.

    The kernels carry the same eight values compiled in; this is the table's
    host-visible form (reference: src/mlx_iqk/nn.py:60-71).
    """
    key = ("vtab", str(torch.device(device) if device is not None else "cpu"))
    if key not in _TABLES:
        _TABLES[key] = torch.from_numpy(IQ2NL_VALUES.astype(np.float16)).to(device or "cpu")
    return _TABLES[key]


def grid_table(device=None) -> torch.Tensor:
    """The IQ1_S grid values as 4096 little-endian uint32 words, two per entry
    (reference: src/mlx_iqk/nn.py:74-88)."""
    key = ("grid", str(torch.device(device) if device is not None else "cpu"))
    if key not in _TABLES:
        words = np.ascontiguousarray(grid_values()).view(np.uint32).reshape(-1).copy()
        _TABLES[key] = torch.from_numpy(words).to(device or "cpu")
    return _TABLES[key]


def member_table(member: str, device=None) -> torch.Tensor:
    check_member(member)
    return grid_table(device) if member == "iq1_s_r4" else value_table(device)


class IqkSwitchLinear(torch.nn.Module):
    """One routed projection: ``num_experts`` IQ_K-quantized ``[out, in]`` matrices
    held as relayout stream buffers, called with ``(x, indices)``."""

    mode = "iqk"
    fused_prefill = True
    """Prefill through the fused contraction (the weights formed inside the
    GEMM, never stored) rather than producer + grouped GEMM.  IQ2_K's are the
    producer's fp16 weights; IQ2_KS and IQ1_S_R4 sum the exact products and
    apply the row scale to the sums, so their weights enter unrounded.  The
    f32 summation order differs too; both routes meet the same float64 gate."""

    def __init__(self, member: str, num_experts: int, out_features: int, in_features: int,
                 device=None):
        super().__init__()
        self.member = check_member(member)
        check_gemv_geometry(in_features, out_features)
        check_dequant_geometry(in_features, out_features)
        self.num_experts = int(num_experts)
        self.out_features = int(out_features)
        self.in_features = int(in_features)
        if self.num_experts <= 0:
            raise IqkRuntimeError(f"a stack needs at least one expert (num_experts={num_experts})")
        dtypes = stream_dtypes(member)
        for name, shape in component_shapes(member, num_experts, out_features, in_features).items():
            self.register_buffer(name, torch.zeros(shape, dtype=dtypes[name], device=device))
        # the streams checked once for the launchers (kernels.CheckedStreams),
        # dropped whenever a stream is reassigned or the module moves, and
        # re-checked whenever a stream's address differs from the record's
        # (register_buffer and ``.data =`` bypass __setattr__)
        names = tuple(component_shapes(member, num_experts, out_features, in_features))
        object.__setattr__(self, "_stream_names", names)
        object.__setattr__(self, "_stream_set", frozenset(names))
        object.__setattr__(self, "_checked_streams", None)
        object.__setattr__(self, "_checked_sig", None)

    def __setattr__(self, name, value):
        if name in self.__dict__.get("_stream_set", ()):
            object.__setattr__(self, "_checked_streams", None)
        super().__setattr__(name, value)

    def _apply(self, fn, *args, **kwargs):
        object.__setattr__(self, "_checked_streams", None)
        return super()._apply(fn, *args, **kwargs)

    def _checked(self) -> kernels.CheckedStreams:
        """The streams as the launchers take them, checked on first use and
        again whenever a stream's address differs from the record's (a new
        tensor; one of another shape or dtype on the same address can only
        be a view of the same storage, which stays allocated)."""
        streams = self._streams()
        sig = [t.data_ptr() for t in streams]
        if self._checked_streams is None or sig != self._checked_sig:
            object.__setattr__(self, "_checked_streams", kernels.CheckedStreams(
                self.member, streams, self.num_experts, self.out_features, self.in_features))
            object.__setattr__(self, "_checked_sig", sig)
        return self._checked_streams

    # -- the relayout streams (module buffers) ---------------------------------

    def stream_names(self) -> list[str]:
        """The member's stream buffer names, ordered as the kernels take them."""
        return list(self._stream_names)

    def _streams(self) -> list[torch.Tensor]:
        buffers = self._buffers  # the stream buffers, without Module.__getattr__'s lookups
        return [buffers[name] for name in self._stream_names]

    def load_streams(self, streams: dict) -> None:
        """Install packed streams (numpy arrays or tensors), checking every shape.

        Arrays land on the module's device with the format's dtypes; a
        missing, extra or misshapen stream is refused
        (reference: src/mlx_iqk/nn.py:137-151).
        """
        shapes = component_shapes(self.member, self.num_experts, self.out_features, self.in_features)
        if set(streams) != set(shapes):
            raise IqkRuntimeError(f"stream set mismatch for {self.member}: expected {sorted(shapes)}, "
                                  f"received {sorted(streams)}")
        dtypes = stream_dtypes(self.member)
        staged = {}
        for name, want in shapes.items():
            value = streams[name]
            if isinstance(value, np.ndarray):
                value = torch.from_numpy(np.ascontiguousarray(value))
            got = tuple(value.shape)
            if got != want:
                raise IqkRuntimeError(
                    f"stream {name} has shape {got}; a {self.num_experts}-expert "
                    f"{self.out_features}x{self.in_features} stack needs {want}")
            if value.dtype != dtypes[name]:
                raise IqkRuntimeError(f"stream {name} must be {dtypes[name]}, got {value.dtype}")
            staged[name] = value
        device = getattr(self, "qs").device
        for name, value in staged.items():
            setattr(self, name, value.to(device).contiguous())

    def load_wire(self, wire: torch.Tensor) -> None:
        """Relayout ik wire rows already on the module's GPU straight into the stream
        buffers (``format.pack`` + :meth:`load_streams`, on the device).  ``wire`` is
        ``u8 [num_experts * out_features, ik_row_bytes]``, experts stacked in order."""
        device = self.qs.device
        rows = self.num_experts * self.out_features
        streams = {k: getattr(self, k).view((rows,) + tuple(getattr(self, k).shape[2:])) for k in self.stream_names()}
        if wire.device != device:
            raise IqkRuntimeError(f"wire is on {wire.device}, the module on {device}")
        if wire.dim() != 2 or int(wire.shape[0]) != rows:
            raise IqkRuntimeError(f"wire must be [{rows}, row bytes], got {tuple(wire.shape)}")
        kernels.pack(self.member, wire.contiguous(), self.in_features, out=streams)

    # -- dequantized route (prefill) -----------------------------------------

    def dequantized(self) -> torch.Tensor:
        """Full fp16 dequantization ``[E, out, in]``, bit-identical to the CPU decode
        (reference: src/mlx_iqk/nn.py:155-169)."""
        return kernels.dequant(self.member, self._checked(), self.num_experts, self.out_features,
                               self.in_features)

    def dequantized_experts(self, slot_of_expert: torch.Tensor, n_slots: int) -> torch.Tensor:
        """fp16 ``[n_slots, out, in]`` holding expert ``e`` in slot ``slot_of_expert[e]``."""
        return kernels.dequant(self.member, self._checked(), self.num_experts, self.out_features,
                               self.in_features, slot_of_expert=slot_of_expert, n_slots=n_slots)

    def dequantized_range(self, start: int, rows: int) -> torch.Tensor:
        """fp16 dequantization of out rows ``[start, start + rows)`` of every
        expert, ``[E, rows, in]``: bit-identical to the same slice of
        :meth:`dequantized` (reference: src/mlx_iqk/nn.py:171-201).  Range-sized
        buffers bound the fp16 memory a sorted prefill holds at once."""
        start, rows = int(start), int(rows)
        self._check_range(start, rows)
        return kernels.dequant(self.member, self._checked(), self.num_experts, self.out_features,
                               self.in_features, row_start=start, rows=rows)

    def _check_range(self, start: int, rows: int) -> None:
        if rows <= 0 or rows & (rows - 1):
            raise IqkRuntimeError(f"a row range spans a power-of-two count of rows, not {rows}")
        if start < 0 or start + rows > self.out_features:
            raise IqkRuntimeError(
                f"rows [{start}, {start + rows}) do not lie within the {self.out_features} rows of an expert")

    # -- call -------------------------------------------------------------------

    def forward(self, x: torch.Tensor, indices: torch.Tensor, sorted_indices: bool = False) -> torch.Tensor:
        """Project ``x`` through the experts named by ``indices`` (route as the reference)."""
        if indices.numel() <= DECODE_MAT_LIMIT and not sorted_indices:
            return self.gemv(x, indices)
        return self.prefill(x, indices)

    def gemv(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        """Fused GEMV over the selected experts; valid for any pair count
        (reference: src/mlx_iqk/nn.py:240-271)."""
        chk = self._checked()
        # Operands already in the kernel's layout (fp16 contiguous x, int32
        # contiguous ids, on the streams' GPU) launch without a reshape and
        # with the output allocated in its final shape: the eager decode's
        # host time is mostly such tensor operations.
        if (x.dtype == torch.float16 and indices.dtype == torch.int32 and chk.gemv_ok
                and x.is_contiguous() and indices.is_contiguous() and x.shape[-1] == self.in_features
                and x.get_device() == chk.device_index and indices.get_device() == chk.device_index):
            mats, rows = indices.numel(), x.numel() // self.in_features
            if rows > 0 and mats % rows == 0:
                out = torch.empty((*indices.shape, 1, self.out_features), dtype=torch.float16, device=chk.device)
                kernels.gemv_checked(self.member, x, chk, indices, rows, mats, out, self.num_experts,
                                     self.out_features)
                return out
        xt = x.reshape(-1, self.in_features)
        if xt.dtype != torch.float16 or not xt.is_contiguous():
            xt = xt.to(torch.float16).contiguous()
        sel = self._device_ids(indices)
        mats, rows = sel.numel(), xt.shape[0]
        # Pairs sharing one activation row: top_k for gate/up, 1 for down.
        if rows <= 0 or mats % rows:
            raise IqkRuntimeError(
                f"{mats} token-expert pairs do not tile {rows} activation row(s); "
                "the operand and the routing disagree")
        out = kernels.gemv(self.member, xt, chk, sel, mats // rows, self.num_experts, self.out_features)
        return out.view(*indices.shape, 1, self.out_features)

    def gemv_sorted(self, x: torch.Tensor, sorted_ids: torch.Tensor, toks: torch.Tensor) -> torch.Tensor:
        """Fused GEMV over expert-sorted pairs, one workgroup per pair
        (reference: src/mlx_iqk/nn.py:273-299).

        Row ``p`` is ``x[toks[p]]`` through expert ``sorted_ids[p]``, each
        element bit-identical to :meth:`gemv`'s for the same pair, so the
        result is the pair GEMV's rows in the caller's sorted order.  IQ2
        members only.
        """
        xt, sel, tok = self._sorted_operands(x, sorted_ids, toks)
        return kernels.gemv_sorted(self.member, xt, self._checked(), sel, tok, self.num_experts,
                                   self.out_features)

    def gemv_union(self, x: torch.Tensor, sorted_ids: torch.Tensor, toks: torch.Tensor) -> torch.Tensor:
        """:meth:`gemv_sorted` decoding each run of equal adjacent ids
        together: the multi-token verify shape, where several pairs select one
        expert (reference: src/mlx_iqk/nn.py:301-333).  Output identical to
        :meth:`gemv_sorted` bit for bit; three adjacent pairs share a
        workgroup, which loads and expands the rows of each run of one expert
        among them once.  The caller applies the inverse permutation."""
        xt, sel, tok = self._sorted_operands(x, sorted_ids, toks)
        return kernels.gemv_sorted(self.member, xt, self._checked(), sel, tok, self.num_experts,
                                   self.out_features, union=True)

    def _device_ids(self, indices: torch.Tensor) -> torch.Tensor:
        """Expert ids as the kernels read them (32-bit, compared unsigned with
        num_experts, so a negative id is out of range).  Wider integers are
        clamped to [-1, num_experts] first, so no out-of-range id wraps into
        the stack."""
        flat = indices.reshape(-1)
        if flat.dtype == torch.int32 and flat.is_contiguous():
            return flat
        if flat.dtype not in (torch.int32, torch.uint32):
            flat = torch.clamp(flat.to(torch.int64), -1, self.num_experts)
        return flat.to(torch.int32).contiguous()

    def _sorted_operands(self, x, sorted_ids, toks):
        xt = x.reshape(-1, self.in_features).to(torch.float16).contiguous()
        sel = self._device_ids(sorted_ids)
        tok = toks.reshape(-1).to(device=sel.device, dtype=torch.int32).contiguous()
        if tok.numel() != sel.numel():
            raise IqkRuntimeError(f"toks carries {tok.numel()} rows for {sel.numel()} pairs")
        return xt, sel, tok

    def prefill(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        """The prefill route of ``forward``: the fused contraction
        (``fused_prefill``, the default), else producer + sorted grouped GEMM.

        Broadcasting follows ``gather_mm(x, W^T, rhs_indices=indices)``: the
        batch shape is ``broadcast(x.shape[:-2], indices.shape)`` and each pair
        contracts its ``x.shape[-2]`` rows.
        """
        return self._sorted_matmul(x, indices, 0, self.out_features)

    def sorted_matmul_range(self, x: torch.Tensor, indices: torch.Tensor, start: int, rows: int) -> torch.Tensor:
        """The sorted dequantized projection over out rows ``[start, start + rows)``
        (reference: src/mlx_iqk/nn.py:203-219): ``[..., M, rows]``.
        Concatenating the ranges along the last axis reproduces
        :meth:`prefill`, element for element (each is the same dot product)."""
        start, rows = int(start), int(rows)
        self._check_range(start, rows)
        return self._sorted_matmul(x, indices, start, rows)

    def _sorted_matmul(self, x: torch.Tensor, indices: torch.Tensor, start: int, rows: int) -> torch.Tensor:
        if x.shape[-1] != self.in_features or x.dim() < 2:
            raise IqkRuntimeError(f"x must be [..., M, {self.in_features}], got {tuple(x.shape)}")
        device = self.qs.device
        xb = x.to(torch.float16)
        M = int(xb.shape[-2])
        batch = torch.broadcast_shapes(tuple(xb.shape[:-2]), tuple(indices.shape))
        P = math.prod(batch)
        if P == 0:
            return torch.empty(tuple(batch) + (M, rows), dtype=torch.float16, device=device)
        xflat = xb.reshape(-1, self.in_features).contiguous()
        E = self.num_experts
        offsets, x_rows, y_rows = self._route(tuple(xb.shape[:-2]), batch, indices, M, xflat.shape[0])
        if self.fused_prefill and self.member in kernels.FUSED_MEMBERS and kernels.fused_fits(
                xflat.shape[0], self.in_features, self.out_features):
            y = kernels.fused_matmul(self.member, xflat, self._checked(), E, self.out_features, offsets, x_rows,
                                     y_rows, row_start=start, rows=rows)
            return y.reshape(tuple(batch) + (M, rows))
        # The producer route: experts are routed only if some pair names them;
        # compact them into slots in expert order (n_slots is an upper bound
        # known on the host) and carry the group offsets over to the slots.
        n_slots = min(E, P)
        present = offsets[1:] > offsets[:-1]
        slot_of_expert = torch.where(present, torch.cumsum(present, 0, dtype=torch.int32) - 1,
                                     torch.full_like(offsets[1:], -1))
        slot_offsets = torch.full((n_slots + 2,), P * M, dtype=torch.int32, device=device)
        slot_offsets.scatter_(0, torch.where(present, slot_of_expert, n_slots + 1).to(torch.int64), offsets[:-1])
        slot_offsets = slot_offsets[:n_slots + 1].contiguous()
        w = kernels.dequant(self.member, self._checked(), E, self.out_features, self.in_features,
                            slot_of_expert=slot_of_expert, n_slots=n_slots, row_start=start, rows=rows)
        y = kernels.grouped_gemm(xflat, w, slot_offsets, x_rows, y_rows)
        return y.reshape(tuple(batch) + (M, rows))

    def _route(self, xbatch: tuple, batch: tuple, indices: torch.Tensor, M: int, n_x_rows: int):
        """Group offsets (per expert, in slots) and each slot's activation and
        output row, slots sorted by expert.  An id outside [0, E) reaches no
        index op (ROCm builds drop torch's device-side bounds asserts): its
        pair is grouped with expert 0 and given an activation row beyond x,
        which the kernels never read and answer with a NaN output row -- what
        the decode route returns."""
        device = self.qs.device
        E = self.num_experts
        # pairs per activation row when x broadcasts over trailing batch dims
        # only (gate/up: x [T, 1, 1, in] with indices [T, k]; sorted pairs:
        # x [P, 1, in] with indices [P]): then one device launch does it all
        pad = (1,) * (len(batch) - len(xbatch)) + tuple(xbatch)
        lead = 0
        while lead < len(batch) and pad[lead] == batch[lead]:
            lead += 1
        if all(d == 1 for d in pad[lead:]) and E <= kernels.ROUTE_MAX_EXPERTS:
            ids = self._device_ids(indices.to(device).broadcast_to(batch))
            return kernels.route(ids, E, M, math.prod(batch[lead:]), n_x_rows)
        xidx = torch.arange(math.prod(xbatch), device=device).reshape(xbatch).broadcast_to(batch).reshape(-1)
        raw = indices.to(device=device, dtype=torch.int64).broadcast_to(batch).reshape(-1)
        valid = (raw >= 0) & (raw < E)
        ids = torch.where(valid, raw, torch.zeros_like(raw))
        order = torch.argsort(ids, stable=True)
        r = torch.arange(M, device=device)
        no_row = torch.full_like(xidx, n_x_rows)
        x_rows = (torch.where(valid, xidx, no_row)[order][:, None] * M + r).reshape(-1)
        x_rows = torch.clamp(x_rows, max=n_x_rows).to(torch.int32)
        y_rows = (order[:, None] * M + r).reshape(-1).to(torch.int32)
        counts = torch.zeros(E, dtype=torch.int64, device=device).index_add_(0, ids, torch.full_like(ids, M))
        offsets = torch.zeros(E + 1, dtype=torch.int32, device=device)
        offsets[1:] = torch.cumsum(counts, 0).to(torch.int32)
        return offsets, x_rows, y_rows


__all__ = ["DECODE_MAT_LIMIT", "IqkKernelError", "IqkRuntimeError", "IqkSwitchLinear", "grid_table",
           "member_table", "value_table"]
