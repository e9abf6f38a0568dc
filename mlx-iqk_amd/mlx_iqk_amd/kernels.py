"""Launch wrappers over the gfx950 kernel library, and their geometry guards.

The reference builds Metal source per geometry and dispatches it through
``mx.fast.metal_kernel`` (src/mlx_iqk/kernels.py:751-887).  Here the kernels
are compiled once into ``libiqk_hip.so``; these wrappers check every tensor
against the geometry on the host, then call the C ABI asynchronously on the
current torch stream.  Nothing here falls back to the CPU: a missing library
raises.

Guards mirror the reference's (src/mlx_iqk/kernels.py:100-142): the decode
GEMV and the producer are sized for input widths 2048 and 4096, the GEMV for
``out_features`` multiples of 16; a width the kernels are not sized for is
refused before anything launches.
"""

from __future__ import annotations

import ctypes

import torch

from . import _native
from .format import MEMBERS, check_member, check_row_width, component_dtypes, component_shapes

IQ2_MEMBERS = ("iq2_ks", "iq2_k")
ROWS_PER_TG = 16
"""Output rows one decode wavefront produces."""
WEIGHTS_PER_LANE = 64
"""Reduction-axis weights each lane of a decode wavefront covers."""
SUPPORTED_IN_FEATURES = (2048, 4096)
DEQUANT_THREADS = 256
TABLE_INPUT_NAMES = {"iq2_ks": "vtab", "iq2_k": "vtab", "iq1_s_r4": "grid"}


class IqkKernelError(RuntimeError):
    pass


def check_gemv_geometry(in_features: int, out_features: int) -> tuple[int, int]:
    n = check_row_width(in_features)
    if n not in SUPPORTED_IN_FEATURES:
        raise IqkKernelError(
            f"no decode GEMV is compiled for in_features={in_features} (widths: {SUPPORTED_IN_FEATURES})")
    out = int(out_features)
    if out <= 0 or out % ROWS_PER_TG:
        raise IqkKernelError(f"the decode GEMV writes rows in tiles of {ROWS_PER_TG}; "
                             f"out_features={out_features} does not fill whole tiles")
    return n, out


def check_dequant_geometry(in_features: int, out_features: int) -> tuple[int, int]:
    n = check_row_width(in_features)
    if n not in SUPPORTED_IN_FEATURES:
        raise IqkKernelError(
            f"no producer is compiled for in_features={in_features} (widths: {SUPPORTED_IN_FEATURES})")
    out = int(out_features)
    if out <= 0:
        raise IqkKernelError(f"out_features must be at least 1, got {out_features}")
    return n, out


def gemv_input_names(member: str) -> list[str]:
    """Input order of a member's decode GEMV (reference: src/mlx_iqk/kernels.py:751-789)."""
    check_member(member)
    return ["x"] + list(component_shapes(member, 1, 1, 2048)) + [TABLE_INPUT_NAMES[member], "sel", "dims"]


def dequant_input_names(member: str) -> list[str]:
    return [n for n in gemv_input_names(member) if n not in ("x", "sel", "dims")]


_TORCH_DTYPES = {"uint8": torch.uint8, "uint16": torch.uint16, "uint32": torch.uint32,
                 "float16": torch.float16}


def stream_dtypes(member: str) -> dict[str, torch.dtype]:
    return {k: _TORCH_DTYPES[v.name] for k, v in component_dtypes(member).items()}


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_ptr(device: torch.device) -> int:
    """The current stream of `device` as a raw stream handle.  torch's raw
    accessor returns the same handle as ``current_stream(device).cuda_stream``
    without building a Stream object (~0.3 against ~2.7 us a call); the public
    call serves where it is absent."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def _require_cuda(t: torch.Tensor, name: str, dtype: torch.dtype | tuple, device=None) -> None:
    if not isinstance(t, torch.Tensor):
        raise IqkKernelError(f"{name} must be a torch tensor")
    if t.device.type != "cuda":
        raise IqkKernelError(f"{name} must live on a GPU, got {t.device}")
    if device is not None and t.device != device:
        raise IqkKernelError(f"{name} is on {t.device}, expected {device}")
    dts = dtype if isinstance(dtype, tuple) else (dtype,)
    if t.dtype not in dts:
        raise IqkKernelError(f"{name} must be {dts}, got {t.dtype}")
    if not t.is_contiguous():
        raise IqkKernelError(f"{name} must be contiguous")


def check_streams(member: str, streams: list[torch.Tensor], num_experts: int, out_features: int,
                  in_features: int) -> torch.device:
    shapes = component_shapes(member, num_experts, out_features, in_features)
    dtypes = stream_dtypes(member)
    if len(streams) != len(shapes):
        raise IqkKernelError(f"{member} needs {len(shapes)} streams, got {len(streams)}")
    device = streams[0].device
    for (name, shape), t in zip(shapes.items(), streams):
        _require_cuda(t, f"stream {name}", dtypes[name], device)
        if tuple(t.shape) != shape:
            raise IqkKernelError(f"stream {name} must be {shape}, got {tuple(t.shape)}")
    return device


class CheckedStreams:
    """A member's streams for one geometry, checked once (count, shapes, dtypes,
    one GPU, contiguity): the device and the pointer array the launchers pass.
    Every launcher takes one in place of the stream list and skips its checks;
    it stays valid while the tensors do (``IqkSwitchLinear`` drops its copy
    whenever a stream is reassigned or the module is moved, and makes a new
    one whenever a stream's address, shape, strides or dtype differ from the
    ones it was made from)."""

    __slots__ = ("key", "device", "device_index", "ptrs", "ptrs_addr", "count", "gemv_ok")

    def __init__(self, member: str, streams: list[torch.Tensor], num_experts: int, out_features: int,
                 in_features: int):
        self.device = check_streams(member, streams, num_experts, out_features, in_features)
        self.device_index = self.device.index if self.device.index is not None else torch.cuda.current_device()
        self.key = (member, int(num_experts), int(out_features), int(in_features))
        self.ptrs = _native.pointer_array([t.data_ptr() for t in streams])
        self.ptrs_addr = ctypes.addressof(self.ptrs)
        self.count = len(streams)
        try:  # a geometry the decode GEMV serves: its launches skip the check
            check_gemv_geometry(in_features, out_features)
            self.gemv_ok = True
        except (IqkKernelError, ValueError):
            self.gemv_ok = False


def _streams_for(member: str, streams, num_experts: int, out_features: int, in_features: int):
    """The device, pointer array and count of a launch's streams: a
    CheckedStreams of this geometry as is, a list checked now."""
    if isinstance(streams, CheckedStreams):
        if streams.key != (member, num_experts, out_features, in_features):
            raise IqkKernelError(f"streams checked for {streams.key}, used for "
                                 f"{(member, num_experts, out_features, in_features)}")
        return streams.device, streams.ptrs, streams.count
    device = check_streams(member, streams, num_experts, out_features, in_features)
    return device, _native.pointer_array([t.data_ptr() for t in streams]), len(streams)


def gemv(member: str, x: torch.Tensor, streams: list[torch.Tensor], sel: torch.Tensor, pairs_per_row: int,
         num_experts: int, out_features: int, *, floor: bool | str = False,
         out: torch.Tensor | None = None) -> torch.Tensor:
    """Decode GEMV: ``y[m] = W[sel[m]] @ x[m // pairs_per_row]``, fp16 ``[mats, out]``.

    ``x`` is fp16 ``[rows, in]``, ``sel`` int32/uint32 ``[mats]`` on the same
    GPU.  ``floor=True`` runs the deleted-decode floor instead, ``floor="grid"``
    that floor with IQ1_S_R4's grid lookups kept (the reference's IQ1 floor).
    """
    n = x.shape[-1]
    if not (isinstance(streams, CheckedStreams) and streams.gemv_ok and streams.key[3] == n):
        check_member(member)
        check_gemv_geometry(n, out_features)
    device, ptrs, n_streams = _streams_for(member, streams, num_experts, out_features, n)
    if not (x.dtype == torch.float16 and x.device == device and x.is_contiguous()):
        _require_cuda(x, "x", torch.float16, device)
    if not (sel.dtype == torch.int32 and sel.device == device and sel.is_contiguous()):
        _require_cuda(sel, "sel", (torch.int32, torch.uint32), device)
    if x.dim() != 2 or sel.dim() != 1:
        raise IqkKernelError("x must be [rows, in_features] and sel [mats]")
    mats = int(sel.numel())
    rows = int(x.shape[0])
    if pairs_per_row <= 0 or rows * pairs_per_row != mats:
        raise IqkKernelError(f"{mats} pairs do not tile {rows} activation rows at {pairs_per_row} per row")
    if out is None:
        out = torch.empty((mats, out_features), dtype=torch.float16, device=device)
    else:
        _require_cuda(out, "out", torch.float16, device)
        if tuple(out.shape) != (mats, out_features):
            raise IqkKernelError(f"out must be {(mats, out_features)}, got {tuple(out.shape)}")
    if mats == 0:
        return out
    kind = 2 if floor == "grid" else 1 if floor else 0
    _gemv_launch(kind, member, n, out_features, num_experts, x.data_ptr(), ptrs, n_streams, sel.data_ptr(),
                 pairs_per_row, mats, out.data_ptr(), _stream_ptr(device))
    return out


def _gemv_launch(kind: int, member: str, n: int, out_features: int, num_experts: int, xp: int, ptrs, n_streams: int,
                 sp: int, pairs_per_row: int, mats: int, yp: int, stream: int) -> None:
    """The launches of :func:`gemv` (kind 0 decode, 1 floor, 2 grid floor) on
    operands already checked: device addresses of x, sel and y, the streams'
    pointer array.  gridDim.y carries the pair index, so the pairs go in
    chunks that keep whole activation rows together."""
    if not 0 < pairs_per_row <= 65535:  # one launch takes at most 65535 pairs
        raise IqkKernelError(f"{pairs_per_row} pairs a row: a decode launch takes 1 .. 65535 pairs of one row")
    fast = _native.launcher()
    lib = None if fast is not None else _native.load()
    ptrs_addr = ctypes.addressof(ptrs)
    limit = (65535 // pairs_per_row) * pairs_per_row
    mid = _native.MEMBER_IDS[member]
    for m0 in range(0, mats, limit):
        cnt = min(limit, mats - m0)
        args = (mid, n, out_features, num_experts, xp + (m0 // pairs_per_row) * n * 2, ptrs_addr, n_streams,
                sp + 4 * m0, pairs_per_row, cnt, yp + m0 * out_features * 2, stream)
        if fast is not None:
            rc = fast.gemv(kind, *args)
        else:
            fn = (lib.iqk_gemv, lib.iqk_gemv_floor, lib.iqk_gemv_floor_grid)[kind]
            rc = fn(*args[:5], ptrs, *args[6:])
        if rc:  # the message is formatted only for a failure
            _native.check(rc, f"iqk_gemv{'_floor' if kind else ''}({member}, {n}x{out_features})")


def gemv_checked(member: str, x: torch.Tensor, streams: "CheckedStreams", sel: torch.Tensor, rows: int, mats: int,
                 out: torch.Tensor, num_experts: int, out_features: int) -> None:
    """The decode GEMV into ``out`` for operands the caller has checked: x
    fp16 and contiguous with ``rows`` rows of the streams' width, sel int32
    and contiguous with ``mats`` ids, out fp16 with ``mats x out_features``
    elements, all on the streams' GPU, ``streams.gemv_ok`` and
    ``mats % rows == 0``.  (The switch module's eager decode path: it skips
    the reshapes and repeated checks of :func:`gemv`.)"""
    if not mats:
        return
    stream = (_raw_stream(streams.device_index) if _raw_stream is not None
              else torch.cuda.current_stream(streams.device).cuda_stream)
    fast = _native.launcher()
    if fast is not None and mats <= 65535:  # one launch: the binding's call with nothing else around it
        rc = fast.gemv(0, _native.MEMBER_IDS[member], streams.key[3], out_features, num_experts, x.data_ptr(),
                       streams.ptrs_addr, streams.count, sel.data_ptr(), mats // rows, mats, out.data_ptr(), stream)
        if rc:
            _native.check(rc, f"iqk_gemv({member}, {streams.key[3]}x{out_features})")
        return
    _gemv_launch(0, member, streams.key[3], out_features, num_experts, x.data_ptr(), streams.ptrs, streams.count,
                 sel.data_ptr(), mats // rows, mats, out.data_ptr(), stream)


def stream_floor_words(nbytes: int, loads: int = 4, max_waves: int = 0) -> int:
    """Output words of :func:`stream_floor` for these arguments."""
    if loads == 4 and not max_waves:
        return (int(nbytes) + 4095) // 4096
    chunks = (int(nbytes) + 1024 * loads - 1) // (1024 * loads)
    waves = min(chunks, max_waves) if max_waves else chunks
    return (waves + 3) // 4 * 4


def stream_floor(src: torch.Tensor, nbytes: int, out: torch.Tensor | None = None, *, loads: int = 4,
                 max_waves: int = 0) -> torch.Tensor:
    """The pure byte-stream floor: one dispatch reading the first ``nbytes`` of
    ``src`` (any contiguous GPU tensor, 16-byte aligned; ``nbytes`` a multiple of
    16), with no expert-id read and no decode.  Returns the dispatch's output
    words (u32, :func:`stream_floor_words` of them, no meaningful values).

    The default form has each wavefront read one 4 KiB chunk; ``loads`` (8 or
    16) puts that many KiB in flight a wavefront, and ``max_waves`` caps the
    wavefronts, which then stride over the span."""
    if not isinstance(src, torch.Tensor) or src.device.type != "cuda" or not src.is_contiguous():
        raise IqkKernelError("src must be a contiguous GPU tensor")
    nbytes, loads, max_waves = int(nbytes), int(loads), int(max_waves)
    if nbytes <= 0 or nbytes % 16 or nbytes > src.numel() * src.element_size():
        raise IqkKernelError(f"{nbytes} bytes is not a positive multiple of 16 within src")
    if loads not in (4, 8, 16) or max_waves < 0:
        raise IqkKernelError(f"loads must be 4, 8 or 16 and max_waves >= 0, got {loads}, {max_waves}")
    words = stream_floor_words(nbytes, loads, max_waves)
    if out is None:
        out = torch.empty(words, dtype=torch.int32, device=src.device)
    elif out.numel() < words or out.dtype not in (torch.int32, torch.uint32) or out.device != src.device:
        raise IqkKernelError(f"out must hold {words} 32-bit words on {src.device}")
    lib = _native.load()
    if loads == 4 and not max_waves:
        rc = lib.iqk_stream_floor(src.data_ptr(), nbytes, out.data_ptr(), _stream_ptr(src.device))
    else:
        rc = lib.iqk_stream_floor_wide(src.data_ptr(), nbytes, loads, max_waves, out.data_ptr(),
                                       _stream_ptr(src.device))
    if rc:
        _native.check(rc, f"iqk_stream_floor({nbytes}, loads={loads}, max_waves={max_waves})")
    return out


def check_iq2_member(member: str) -> str:
    """Members the sorted and union GEMVs cover (reference: src/mlx_iqk/kernels.py:89-97)."""
    check_member(member)
    if member not in IQ2_MEMBERS:
        raise IqkKernelError(
            f"{member!r} has no expert-sorted GEMV; those forms exist for {IQ2_MEMBERS}")
    return member


def gemv_sorted(member: str, x: torch.Tensor, streams: list[torch.Tensor], sorted_ids: torch.Tensor,
                toks: torch.Tensor, num_experts: int, out_features: int, *, union: bool = False,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """Decode GEMV over expert-sorted pairs: ``y[p] = W[sorted_ids[p]] @ x[toks[p]]``.

    fp16 ``[mats, out]``; each element equals :func:`gemv`'s for the same
    (expert, activation row), bit for bit.  ``union=True`` is the union entry
    point (the multi-token verify shape, src/mlx_iqk/kernels.py:484-578),
    otherwise the sorted one (src/mlx_iqk/kernels.py:404-482).  The sorted
    form runs one workgroup per pair; the union form gives three adjacent
    pairs a workgroup, which loads and expands the rows of each run of one
    expert among them once.  IQ2 members only.
    """
    check_iq2_member(member)
    n = int(x.shape[-1])
    check_gemv_geometry(n, out_features)
    device, ptrs, n_streams = _streams_for(member, streams, num_experts, out_features, n)
    _require_cuda(x, "x", torch.float16, device)
    _require_cuda(sorted_ids, "sorted_ids", (torch.int32, torch.uint32), device)
    _require_cuda(toks, "toks", (torch.int32, torch.uint32), device)
    if x.dim() != 2 or sorted_ids.dim() != 1 or toks.dim() != 1:
        raise IqkKernelError("x must be [rows, in_features], sorted_ids and toks [mats]")
    mats = int(sorted_ids.numel())
    if int(toks.numel()) != mats:
        raise IqkKernelError(f"toks carries {int(toks.numel())} rows for {mats} pairs")
    if out is None:
        out = torch.empty((mats, out_features), dtype=torch.float16, device=device)
    else:
        _require_cuda(out, "out", torch.float16, device)
        if tuple(out.shape) != (mats, out_features):
            raise IqkKernelError(f"out must be {(mats, out_features)}, got {tuple(out.shape)}")
    if mats == 0:
        return out
    lib = _native.load()
    fn = lib.iqk_gemv_union if union else lib.iqk_gemv_sorted
    stream = _stream_ptr(device)
    # The pair index rides gridDim.z: chunks of at most 65535 pairs.  A run of
    # equal ids split by a chunk boundary is read once per chunk.
    for m0 in range(0, mats, 65535):
        cnt = min(65535, mats - m0)
        rc = fn(_native.MEMBER_IDS[member], n, out_features, num_experts, x.data_ptr(), int(x.shape[0]), ptrs,
                n_streams, sorted_ids.data_ptr() + 4 * m0, toks.data_ptr() + 4 * m0, cnt,
                out.data_ptr() + m0 * out_features * 2, stream)
        if rc:
            _native.check(rc, f"iqk_gemv_{'union' if union else 'sorted'}({member}, {n}x{out_features})")
    return out


def dequant(member: str, streams: list[torch.Tensor], num_experts: int, out_features: int, in_features: int,
            *, slot_of_expert: torch.Tensor | None = None, n_slots: int | None = None, floor: bool = False,
            row_start: int = 0, rows: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Producer: fp16 ``[n_slots, rows, in]``, slot ``slot_of_expert[e]`` <- rows
    ``[row_start, row_start + rows)`` of expert ``e`` (default: every row).

    Without ``slot_of_expert`` every expert lands in its own slot.  Slots no
    expert maps to are left unwritten.  A row range is bit-identical to the
    same slice of the full reconstruction.
    """
    check_member(member)
    check_dequant_geometry(in_features, out_features)
    row_start = int(row_start)
    rows = out_features - row_start if rows is None else int(rows)
    ranged = row_start != 0 or rows != out_features
    if row_start < 0 or rows <= 0 or row_start + rows > out_features:
        raise IqkKernelError(f"row range [{row_start}, {row_start + rows}) is outside out_features {out_features}")
    if floor and (row_start or rows != out_features):
        raise IqkKernelError("the producer's floor covers full experts only")
    device, ptrs, n_streams = _streams_for(member, streams, num_experts, out_features, in_features)
    if slot_of_expert is None:
        n_slots = num_experts if n_slots is None else int(n_slots)
        if n_slots < num_experts:
            raise IqkKernelError("without slot_of_expert every expert needs its own slot")
        slot_ptr = None
    else:
        _require_cuda(slot_of_expert, "slot_of_expert", torch.int32, device)
        if tuple(slot_of_expert.shape) != (num_experts,):
            raise IqkKernelError(f"slot_of_expert must be [{num_experts}]")
        if n_slots is None:
            raise IqkKernelError("n_slots is required with slot_of_expert")
        slot_ptr = slot_of_expert.data_ptr()
    shape = (int(n_slots), rows, in_features)
    if out is None:
        out = torch.empty(shape, dtype=torch.float16, device=device)
    else:
        _require_cuda(out, "out", torch.float16, device)
        if tuple(out.shape) != shape:
            raise IqkKernelError(f"out must be {shape}, got {tuple(out.shape)}")
    lib = _native.load()
    mid = _native.MEMBER_IDS[member]
    if ranged:
        rc = lib.iqk_dequant_rows(mid, in_features, out_features, num_experts, ptrs, n_streams, row_start,
                                  rows, slot_ptr, int(n_slots), out.data_ptr(), _stream_ptr(device))
        if rc:
            _native.check(rc, f"iqk_dequant_rows({member}, {in_features}x{out_features}, [{row_start}, +{rows}))")
        return out
    fn = lib.iqk_dequant_floor if floor else lib.iqk_dequant
    rc = fn(mid, in_features, out_features, num_experts, ptrs, n_streams,
            slot_ptr, int(n_slots), out.data_ptr(), _stream_ptr(device))
    if rc:
        _native.check(rc, f"iqk_dequant{'_floor' if floor else ''}({member}, {in_features}x{out_features})")
    return out


def grouped_gemm(x: torch.Tensor, w: torch.Tensor, group_offsets: torch.Tensor, x_rows: torch.Tensor,
                 y_rows: torch.Tensor | None = None, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """Sorted grouped GEMM: ``y[y_rows[p]] = x[x_rows[p]] @ w[g(p)]^T`` for slot ``p``.

    ``x`` fp16 ``[rows, K]``; ``w`` fp16 ``[G, N, K]``; ``group_offsets``
    int32 ``[G + 1]`` (slot ranges, sorted by group); ``x_rows``/``y_rows``
    int32 ``[P]``.  Returns fp16 ``[P, N]``.
    """
    _require_cuda(x, "x", torch.float16)
    device = x.device
    _require_cuda(w, "w", torch.float16, device)
    _require_cuda(group_offsets, "group_offsets", (torch.int32, torch.uint32), device)
    _require_cuda(x_rows, "x_rows", (torch.int32, torch.uint32), device)
    if x.dim() != 2 or w.dim() != 3 or w.shape[2] != x.shape[1]:
        raise IqkKernelError(f"x [rows, K] and w [G, N, K] disagree: {tuple(x.shape)} vs {tuple(w.shape)}")
    G, N, K = (int(s) for s in w.shape)
    P = int(x_rows.numel())
    if tuple(group_offsets.shape) != (G + 1,):
        raise IqkKernelError(f"group_offsets must be [{G + 1}]")
    if N <= 0 or K % 32:
        raise IqkKernelError(f"grouped gemm needs N > 0 and K % 32 == 0, got N={N}, K={K}")
    if y_rows is not None:
        _require_cuda(y_rows, "y_rows", (torch.int32, torch.uint32), device)
        if y_rows.numel() != P:
            raise IqkKernelError("y_rows and x_rows must have the same length")
    if out is None:
        out = torch.empty((P, N), dtype=torch.float16, device=device)
    else:
        _require_cuda(out, "out", torch.float16, device)
        if tuple(out.shape) != (P, N):
            raise IqkKernelError(f"out must be {(P, N)}")
    rc = _native.load().iqk_grouped_gemm(
        K, N, G, P, x.data_ptr(), int(x.shape[0]), w.data_ptr(), group_offsets.data_ptr(), x_rows.data_ptr(),
        y_rows.data_ptr() if y_rows is not None else None, out.data_ptr(), _stream_ptr(device))
    if rc:
        _native.check(rc, f"iqk_grouped_gemm(K={K}, N={N}, G={G}, P={P})")
    return out


def pack(member: str, wire: torch.Tensor, in_features: int,
         out: dict[str, torch.Tensor] | None = None) -> dict[str, torch.Tensor]:
    """``format.pack`` on the GPU: ik wire rows ``u8 [rows, ik_row_bytes]`` already in
    device memory -> the member's relayout streams (``[rows, ...]`` each), bit for bit.
    ``out`` may hold the destination planes (e.g. views of a module's buffers)."""
    from .format import check_wire_rows, ik_row_bytes
    check_member(member)
    n = check_row_width(in_features, member)
    _require_cuda(wire, "wire", torch.uint8)
    rows = int(wire.shape[0]) if wire.dim() == 2 else -1
    if wire.dim() != 2 or int(wire.shape[1]) != ik_row_bytes(member, n):
        raise IqkKernelError(f"{member} wire rows of {n} weights are {ik_row_bytes(member, n)} bytes, "
                             f"got {tuple(wire.shape)}")
    check_wire_rows(member, rows)
    shapes = {k: v[1:] for k, v in component_shapes(member, 1, rows, n).items()}
    dtypes = stream_dtypes(member)
    if out is None:
        out = {k: torch.empty(shape, dtype=dtypes[k], device=wire.device) for k, shape in shapes.items()}
    else:
        for k, shape in shapes.items():
            _require_cuda(out[k], f"stream {k}", dtypes[k], wire.device)
            if tuple(out[k].shape) != shape:
                raise IqkKernelError(f"stream {k} must be {shape}, got {tuple(out[k].shape)}")
    if rows == 0:
        return out
    ptrs = _native.pointer_array([out[k].data_ptr() for k in shapes])
    rc = _native.load().iqk_pack(_native.MEMBER_IDS[member], n, rows, wire.data_ptr(), ptrs, len(shapes),
                                 _stream_ptr(wire.device))
    if rc:
        _native.check(rc, f"iqk_pack({member}, {n}, rows={rows})")
    return out


ROUTE_MAX_EXPERTS = 4096
"""Stacks the device-side route serves (its counters live in LDS)."""


def route(ids: torch.Tensor, num_experts: int, rows_per_pair: int = 1, pairs_per_x_row: int = 1,
          n_x_rows: int | None = None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Expert-sorted slots of token-expert pairs, on the device, one launch.

    ``ids`` int32/uint32 ``[P]``: pair p's expert (an id outside
    ``[0, num_experts)``, read as u32, is grouped with expert 0 and given no
    activation row, so the prefill kernels answer it with NaN rows).  Pair p
    owns ``rows_per_pair`` slots whose activation rows are
    ``(p // pairs_per_x_row) * rows_per_pair + r`` and output rows
    ``p * rows_per_pair + r``.  Returns int32 ``group_offsets [E + 1]``,
    ``x_rows [P * rows_per_pair]``, ``y_rows [P * rows_per_pair]``; the slot
    order is stable (pairs keep their order within an expert).
    """
    _require_cuda(ids, "ids", (torch.int32, torch.uint32))
    if ids.dim() != 1:
        raise IqkKernelError("ids must be [pairs]")
    E, P, M, ppx = int(num_experts), int(ids.numel()), int(rows_per_pair), int(pairs_per_x_row)
    if not 0 < E <= ROUTE_MAX_EXPERTS:
        raise IqkKernelError(f"the device route serves 1 .. {ROUTE_MAX_EXPERTS} experts, got {E}")
    if M <= 0 or ppx <= 0:
        raise IqkKernelError("rows_per_pair and pairs_per_x_row must be positive")
    rows = ((P + ppx - 1) // ppx) * M if n_x_rows is None else int(n_x_rows)
    offs = torch.empty(E + 1, dtype=torch.int32, device=ids.device)
    x_rows = torch.empty(P * M, dtype=torch.int32, device=ids.device)
    y_rows = torch.empty(P * M, dtype=torch.int32, device=ids.device)
    rc = _native.load().iqk_route(ids.data_ptr(), P, E, M, ppx, rows, offs.data_ptr(), x_rows.data_ptr(),
                                  y_rows.data_ptr(), _stream_ptr(ids.device))
    if rc:
        _native.check(rc, f"iqk_route(P={P}, E={E}, M={M})")
    return offs, x_rows, y_rows


FUSED_MEMBERS = MEMBERS
"""Members the fused prefill contraction covers (all three)."""


def fused_fits(n_x_rows: int, in_features: int, out_features: int) -> bool:
    """Whether the fused prefill serves these operands: its lane offsets are
    32-bit, within one expert's code plane (``in/4`` bytes a row) and within
    x, so both stay below 4 GiB (the entry point refuses larger ones)."""
    return out_features * (in_features // 4) < 1 << 32 and 0 < n_x_rows and n_x_rows * in_features * 2 < 1 << 32


def fused_matmul(member: str, x: torch.Tensor, streams: list[torch.Tensor], num_experts: int, out_features: int,
                 group_offsets: torch.Tensor, x_rows: torch.Tensor, y_rows: torch.Tensor | None = None, *,
                 row_start: int = 0, rows: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Prefill contraction straight from the streams: ``y[y_rows[p]] = x[x_rows[p]] @ W[e, r0:r0+rows]^T``
    for the slots ``p`` of expert ``e`` (``[group_offsets[e], group_offsets[e+1])``), with
    ``W`` formed inside the GEMM: IQ2_K's as the producer's fp16 weights, IQ2_KS's and
    IQ1_S_R4's as exact products whose row scale multiplies the f32 sums.  fp16 ``[P, rows]``."""
    if member not in FUSED_MEMBERS:
        raise IqkKernelError(f"the fused prefill covers {FUSED_MEMBERS}; {member!r} takes the producer route")
    n = int(x.shape[-1])
    check_dequant_geometry(n, out_features)
    row_start = int(row_start)
    rows = out_features - row_start if rows is None else int(rows)
    if row_start < 0 or rows <= 0 or row_start + rows > out_features:
        raise IqkKernelError(f"row range [{row_start}, {row_start + rows}) is outside out_features {out_features}")
    device, ptrs, n_streams = _streams_for(member, streams, num_experts, out_features, n)
    _require_cuda(x, "x", torch.float16, device)
    _require_cuda(group_offsets, "group_offsets", (torch.int32, torch.uint32), device)
    _require_cuda(x_rows, "x_rows", (torch.int32, torch.uint32), device)
    if x.dim() != 2 or tuple(group_offsets.shape) != (num_experts + 1,):
        raise IqkKernelError(f"x must be [rows, {n}] and group_offsets [{num_experts + 1}]")
    P = int(x_rows.numel())
    if y_rows is not None:
        _require_cuda(y_rows, "y_rows", (torch.int32, torch.uint32), device)
        if y_rows.numel() != P:
            raise IqkKernelError("y_rows and x_rows must have the same length")
    if out is None:
        out = torch.empty((P, rows), dtype=torch.float16, device=device)
    else:
        _require_cuda(out, "out", torch.float16, device)
        if tuple(out.shape) != (P, rows):
            raise IqkKernelError(f"out must be {(P, rows)}")
    rc = _native.load().iqk_fused_gemm(
        _native.MEMBER_IDS[member], n, out_features, num_experts, x.data_ptr(), int(x.shape[0]), ptrs, n_streams,
        row_start, rows, group_offsets.data_ptr(), x_rows.data_ptr(), y_rows.data_ptr() if y_rows is not None else None, P,
        out.data_ptr(), _stream_ptr(device))
    if rc:
        _native.check(rc, f"iqk_fused_gemm({member}, {n}x{out_features}, P={P})")
    return out


__all__ = [
    "DEQUANT_THREADS", "IQ2_MEMBERS", "MEMBERS", "ROWS_PER_TG",
    "SUPPORTED_IN_FEATURES", "TABLE_INPUT_NAMES", "WEIGHTS_PER_LANE", "IqkKernelError",
    "check_dequant_geometry", "check_gemv_geometry", "check_streams", "dequant", "dequant_input_names",
    "CheckedStreams", "FUSED_MEMBERS", "ROUTE_MAX_EXPERTS", "check_iq2_member", "fused_fits", "fused_matmul", "gemv", "pack", "route", "stream_floor", "gemv_input_names", "gemv_sorted", "grouped_gemm",
    "stream_dtypes",
]
