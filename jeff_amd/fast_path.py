"""The fast path's fused linear layer on MI355X: Lin, Workspace, lora_add, the stacked adapter pool.

Mirrors the reference's engine/fast_path.py (paths relative to runtime/python/src/jeff_runtime/):
- Lin (fast_path.py:301-349): matrices that read the same input, fused along the output, with their LoRA updates in
  every adapter's row of a stacked pool. Differences, each for the MI355X kernels:
  * each matrix j has its own rank capacity cap_j (default 16 for an adapted matrix, as the reference gives each
    one) and every adapter its own live rank r <= cap_j per matrix, held in a device table; the kernels read only
    the live ranks, so rank-8 and rank-64 adapters share a pool without padding reads;
  * the second factor is stored per matrix as sB_j (out_j, s) instead of one block-diagonal Bt (rank, out): no
    zero blocks in HBM, and each output column's rank vector is one contiguous 16-byte read for the MFMA operand.
    The row stride s is the adapter's live rank rounded up to a power of two (at least 8, at most cap_j, `sb_stride`),
    so a low-rank adapter's sB is dense: the block reserves out_j * cap_j elements and the adapter fills the first
    out_j * s of them.
  The first factors keep the reference layout: A (rank, k) at off_a, matrix j in rows [rho_j, rho_j + cap_j).
- Workspace (fast_path.py:261-274): per pass shape, the scratch the products share: the LoRA first factors (mid,
  bf16, tokens x rank) and the routed pass (the sorted order of the request rows by adapter).
- lora_add (fast_path.py:277-289): y += bf16(x A^T) sB^T in place, per token's adapter row.
- AdapterPool (FastPath.lora_pool / add_adapter / remove_adapter / index, fast_path.py:456-547): row 0 is the base
  (no update), adapters take the lowest free row, removal frees the row (its live ranks set to 0, so no kernel reads
  it again).
Everything on the GPU runs in the HIP library (jeff_amd/libjeff_mlora.so); there is no PyTorch fallback."""

from __future__ import annotations

import bisect
import weakref
from collections.abc import Callable, Mapping, Sequence
from dataclasses import dataclass

import torch

from jeff_amd import _lib
from jeff_amd.int4 import KernelInt4

DT = torch.bfloat16
# The matrices an adapter may adapt, by the last part of the layer name (fast_path.py:68-69), plus their HF names
LORA_TARGETS = ("in_proj_qkv", "in_proj_z", "out_proj", "q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj",
                "down_proj")
DEFAULT_RANK = 16  # per adapted matrix, as the reference's fast path (fast_path.py:316)

Update = tuple[torch.Tensor, torch.Tensor]  # (A (r, in), sB (out, r)): the scale alpha / r already folded into B


def sb_stride(rank: int, cap: int) -> int:
    """Row stride of an adapter's sB_j in the pool: its live rank rounded up to a power of two, at least 8, at most
    cap_j (jeff_amd/csrc/mlora_common.h sb_stride; a rank-0 row keeps min(8, cap_j))."""
    s = 8
    while s < rank:
        s *= 2
    return min(s, cap)


def fold_scale(b: torch.Tensor, scale: float, dtype: torch.dtype = DT) -> torch.Tensor:
    """engine/lora.py:209-210: s*B, multiplied in float32, then cast to the model's dtype."""
    return (b.to(torch.float32) * scale).to(dtype).contiguous()


class Lin:
    """A fused group (fast_path.py:301-349). `weights`: the matrices' bf16 (out_j, k) weights, or None with `sizes`
    and `k` for a group that only has INT4 weights (attach `int4`). `ranks`: each matrix's rank capacity (a multiple of
    8), default 16 for a matrix whose name ends in one of LORA_TARGETS and 0 otherwise."""

    def __init__(self, names: list[str], weights: list[torch.Tensor] | None = None, *,
                 sizes: Sequence[int] | None = None, k: int | None = None,
                 ranks: Sequence[int] | None = None) -> None:
        if len(names) > _lib.MAX_MATS or not names:
            raise ValueError(f"A fused group holds 1 to {_lib.MAX_MATS} matrices; got {len(names)}")
        self.names = list(names)
        if weights is not None:
            self.sizes = [int(w.shape[0]) for w in weights]
            self.k = int(weights[0].shape[1])
            self.W: torch.Tensor | None = torch.cat(list(weights)).to(DT).contiguous()
        else:
            if sizes is None or k is None:
                raise ValueError("Lin needs the weights, or the matrices' sizes and inputs")
            self.sizes = [int(s) for s in sizes]
            self.k = int(k)
            self.W = None
        if len(self.sizes) != len(self.names):
            raise ValueError("one size per matrix name")
        self.out = sum(self.sizes)
        if ranks is None:
            ranks = [DEFAULT_RANK if n.rsplit(".", 1)[-1] in LORA_TARGETS else 0 for n in self.names]
        self.caps = [int(r) for r in ranks]
        if len(self.caps) != len(self.names) or any(r < 0 or r % 8 for r in self.caps):
            raise ValueError(f"{', '.join(self.names)}: rank capacities must be multiples of 8, one per matrix; got "
                             f"{list(ranks)}")
        self.rank = sum(self.caps)
        self.rho = [sum(self.caps[:j]) for j in range(len(self.caps))]
        self.cols0 = [sum(self.sizes[:j]) for j in range(len(self.sizes))]
        self.pool: torch.Tensor
        self.ranks_table: torch.Tensor
        self.rank_col = 0
        self.off_a = self.off_b = 0
        self.off_bj: list[int] = []
        self.int4: KernelInt4 | None = None

    def numel(self) -> int:
        """Pool elements per adapter row: A (rank, k) plus sB_j (out_j, cap_j) for every matrix."""
        return self.rank * self.k + sum(n * c for n, c in zip(self.sizes, self.caps))

    def bind(self, pool: torch.Tensor, offset: int, ranks_table: torch.Tensor | None = None,
             rank_col: int = 0) -> None:
        """Read this group's LoRA matrices at `offset` in every row of the stacked pool; its live ranks in columns
        rank_col.. of ranks_table (int32, one row per pool row; a zero table when None)."""
        if offset % 8 or pool.stride(0) % 8 or pool.dtype != DT:
            raise ValueError("the pool must be bf16 with 16-byte aligned rows and offsets")
        self.pool = pool
        self.off_a = offset
        self.off_b = offset + self.rank * self.k
        self.off_bj = [self.off_b + sum(n * c for n, c in zip(self.sizes[:j], self.caps[:j]))
                       for j in range(len(self.sizes))]
        if ranks_table is None:
            ranks_table = torch.zeros(pool.shape[0], len(self.names), dtype=torch.int32, device=pool.device)
        self.ranks_table = ranks_table
        self.rank_col = rank_col

    def pack(self, flat: torch.Tensor, updates: Mapping[str, Update]) -> list[int]:
        """Write one adapter's updates {matrix name: (A (r, in), sB (out, r))} into this group's slice of `flat` (all
        zeros before); returns the live rank of each matrix (0 for a matrix without an update)."""
        a_view = flat[:self.rank * self.k].view(self.rank, self.k)
        live = []
        for j, (name, size, cap) in enumerate(zip(self.names, self.sizes, self.caps, strict=True)):
            if name not in updates:
                live.append(0)
                continue
            a, sb = updates[name]
            r = int(a.shape[0])
            if r > cap:
                raise ValueError(f"{name}: LoRA rank {r} does not fit the fast path's rank-{cap} buffer")
            if tuple(a.shape) != (r, self.k) or tuple(sb.shape) != (size, r):
                raise ValueError(f"{name}: LoRA shapes {tuple(a.shape)} and {tuple(sb.shape)} do not fit a "
                                 f"({size}, {self.k}) layer")
            a_view[self.rho[j]:self.rho[j] + r] = a
            start = self.off_bj[j] - self.off_a
            stride = sb_stride(r, cap)
            b_view = flat[start:start + size * stride].view(size, stride)
            b_view[:, :r] = sb
            live.append(r)
        return live

    def lora_abi(self) -> _lib.Lora:
        """The C description of this group's pool slice (pointers stay valid while the pool lives)."""
        n = len(self.names)
        off_b = (_lib.c_i64 * _lib.MAX_MATS)(*(self.off_bj + [0] * (_lib.MAX_MATS - n)))
        cap = (_lib.c_i32 * _lib.MAX_MATS)(*(self.caps + [0] * (_lib.MAX_MATS - n)))
        cols = (_lib.c_i32 * _lib.MAX_MATS)(*(self.sizes + [0] * (_lib.MAX_MATS - n)))
        ranks = self.ranks_table
        return _lib.Lora(self.pool.data_ptr(), ranks.data_ptr() + 4 * self.rank_col, self.pool.stride(0), self.off_a,
                         off_b, ranks.stride(0), self.pool.shape[0], n, self.rank, cap, cols)

    def __call__(self, x: torch.Tensor, ws: Workspace, adp: torch.Tensor) -> torch.Tensor:
        """fast_path.py:347-349: the fused product of x through the bf16 W (torch's library GEMM) plus each token's
        adapter update (lora_add)."""
        if self.W is None:
            raise ValueError(f"{', '.join(self.names)}: no bfloat16 weights (an INT4-only group runs int4_product)")
        return lora_add(x @ self.W.T, x, self, adp, ws)


@dataclass(frozen=True)
class RouteRecord:
    """What the last routing launch of a workspace routed: the adp tensor (by identity) and its version, the pass's
    sizes, the cu_seqlens tensor and version (None for uniform rows), the stream and the graph capture it went to
    (HIP's capture sequence id, 0 outside a capture)."""
    adp: Callable[[], torch.Tensor | None]
    adp_version: int
    requests: int
    tokens: int
    pool_rows: int
    cu: Callable[[], torch.Tensor | None] | None
    cu_version: int
    stream: int
    capture: int


def reusable(last: RouteRecord, adp: torch.Tensor, tokens: int, pool_rows: int, stream: int, capture: int) -> bool:
    """Whether a product may read the route `last` describes instead of routing again: only inside the graph capture
    that recorded that routing launch (so every replay runs it first), on the same stream, for the same adp tensor
    object unchanged since (its version counter; a new tensor at a reused address is another object) and unchanged
    cu_seqlens. Outside a capture a product always routes again: graph replays of the same workspace are invisible
    to Python and may have overwritten the route with another pass's since."""
    if capture == 0 or last.capture != capture or last.stream != stream:
        return False
    if last.adp() is not adp or last.adp_version != adp._version or last.requests != adp.numel():
        return False
    if last.tokens != tokens or last.pool_rows != pool_rows:
        return False
    if last.cu is not None:
        cu = last.cu()
        if cu is None or cu._version != last.cu_version:
            return False
    return True


class Workspace:
    """fast_path.py:261-274: scratch shared by the products of passes of up to `rows` tokens in request rows of
    `row_len` tokens (uniform rows, as the reference's passes), or ragged rows routed with cu_seqlens.
    `shapes`: the (k, out) of the groups that will run: the float32 partials of their split and narrow products are
    allocated here, up front, at the most any of them needs for up to `rows` tokens (mlora_int4_partials_bound), as
    the reference sizes its QP from the shapes; `max_rank`: the largest stacked rank capacity (Lin.rank) of those
    groups; `max_requests`: request rows per pass (default rows/row_len)."""

    def __init__(self, rows: int, row_len: int, shapes: set[tuple[int, int]] | None = None, *, max_rank: int = 256,
                 max_requests: int | None = None, device: torch.device | str = "cuda") -> None:
        if row_len <= 0 or rows % row_len:
            raise ValueError(f"A workspace of {rows} tokens cannot hold whole rows of {row_len} tokens")
        self.rows = rows
        self.row_len = row_len
        self.shapes = set(shapes or ())
        self.max_rank = max_rank
        self.max_requests = max_requests if max_requests is not None else rows // row_len
        if self.max_requests > _lib.MAX_REQUESTS:
            raise ValueError(f"{self.max_requests} request rows per pass; the routing kernel sorts at most "
                             f"{_lib.MAX_REQUESTS}")
        h = _lib.lib()
        dev = torch.device(device)
        nbytes = h.mlora_workspace_bytes(rows, max_rank)
        self.mid = torch.empty(nbytes // 2, dtype=DT, device=dev)
        b = max(self.max_requests, 1)
        i32 = dict(dtype=torch.int32, device=dev)
        self.req_order = torch.empty(b, **i32)
        self.tok_perm = torch.empty(max(rows, 1), **i32)
        self.last_of = torch.empty(max(rows, 1), **i32)
        self.seg_of = torch.empty(max(rows, 1), **i32)
        self.seg_start = torch.empty(b + 1, **i32)
        self.seg_adapter = torch.empty(b, **i32)
        self.num_segs = torch.zeros(1, **i32)
        self.status = torch.zeros(1, **i32)
        self._last: RouteRecord | None = None
        self._route_abi: _lib.Route | None = None
        self._part: torch.Tensor | None = None
        self._retired: list[torch.Tensor] = []
        bound = max((h.mlora_int4_partials_bound(k, -(-out // 64) * 64, out, rows) for k, out in self.shapes),
                    default=0)
        if bound:
            self._part = torch.empty(bound, dtype=torch.uint8, device=dev)

    def partials(self, nbytes: int) -> tuple[int, int]:
        """(pointer, bytes) of device scratch for a split or narrow product's float32 partial sums, at least nbytes
        (0: none needed). The buffer sized from `shapes` serves every product of those shapes; a product that needs more
        (a shape not named, or kernels forced by flags) gets a larger buffer, and the smaller one is kept alive with the
        workspace, never freed: a graph recorded earlier holds its address and writes it on every replay (the reference
        allocates its partials per product instead, engine/int4_kernels.py:160-166)."""
        if nbytes == 0:
            return 0, 0
        if self._part is None or self._part.numel() < nbytes:
            if self._part is not None:
                self._retired.append(self._part)
            self._part = torch.empty(nbytes, dtype=torch.uint8, device=self.mid.device)
        return self._part.data_ptr(), self._part.numel()

    def route(self, adp: torch.Tensor, pool_rows: int, tokens: int | None = None,
              cu_seqlens: torch.Tensor | None = None) -> _lib.Route:
        """Sort this pass's request rows by adapter index: one launch on the current stream, every call. Uniform
        rows: tokens = len(adp) * row_len. Ragged rows: cu_seqlens int32 (requests + 1) on the device and `tokens`
        (its last value) given by the caller, since reading it would synchronise. The products that follow with the
        same adp route it again the same way (with these cu_seqlens), or, inside one graph capture, share this
        launch (routed)."""
        requests = int(adp.numel())
        if adp.dtype != torch.int32 or adp.device.type != "cuda" or not adp.is_contiguous():
            raise ValueError("adp must be a contiguous int32 tensor on the GPU")
        if requests > self.max_requests:
            raise ValueError(f"{requests} request rows; this workspace routes at most {self.max_requests}")
        if cu_seqlens is None:
            tokens = requests * self.row_len if tokens is None else tokens
            if tokens != requests * self.row_len:
                raise ValueError(f"{tokens} tokens are not {requests} rows of {self.row_len}")
        else:
            if tokens is None:
                raise ValueError("ragged rows need the token count (cu_seqlens[-1]) from the caller")
            if cu_seqlens.dtype != torch.int32 or cu_seqlens.numel() != requests + 1 or not cu_seqlens.is_contiguous():
                raise ValueError("cu_seqlens must be a contiguous int32 tensor of requests + 1 offsets")
        if tokens > self.rows:
            raise ValueError(f"A pass of {tokens} tokens does not fit a workspace of {self.rows}")
        r = _lib.Route(self.req_order.data_ptr(), self.tok_perm.data_ptr(), self.last_of.data_ptr(),
                       self.seg_of.data_ptr(), self.seg_start.data_ptr(), self.seg_adapter.data_ptr(),
                       self.num_segs.data_ptr(), self.status.data_ptr(), tokens, requests,
                       max(min(requests, pool_rows), 1))
        h = _lib.lib()
        stream = torch.cuda.current_stream(adp.device).cuda_stream
        _lib.check(h.mlora_route(adp.data_ptr(), 0 if cu_seqlens is None else cu_seqlens.data_ptr(),
                                 0 if cu_seqlens is not None else self.row_len, r, pool_rows, stream), "mlora_route")
        self._last = RouteRecord(weakref.ref(adp), adp._version, requests, tokens, pool_rows,
                                 None if cu_seqlens is None else weakref.ref(cu_seqlens),
                                 -1 if cu_seqlens is None else cu_seqlens._version, stream, _lib.capture_id(stream))
        self._route_abi = r
        return r

    def routed(self, adp: torch.Tensor, pool_rows: int, tokens: int) -> _lib.Route:
        """The route a product of `tokens` tokens over `adp` reads. Inside a graph capture, the route launched
        earlier in the same capture for this very adp tensor (unchanged since, same stream) is shared: the graph
        replays that launch before this product. Otherwise the route is launched again, with the cu_seqlens of the
        last ws.route of this adp when there was one (ragged rows), else over uniform rows of row_len."""
        last = self._last
        stream = torch.cuda.current_stream(adp.device).cuda_stream
        capture = _lib.capture_id(stream)
        if last is not None and reusable(last, adp, tokens, pool_rows, stream, capture):
            return self._route_abi
        cu = None
        if last is not None and last.adp() is adp and last.cu is not None:
            cu = last.cu()
        return self.route(adp, pool_rows, tokens=tokens, cu_seqlens=cu)

    def check(self) -> None:
        """Raise ValueError if the last routing met an adapter index out of range or unusable cu_seqlens (reads the
        device status: synchronises)."""
        s = int(self.status.item())
        if s & _lib.ROUTE_BAD_ADAPTER:
            raise ValueError("an adapter index lay outside the pool; those rows were served by the base (row 0)")
        if s & _lib.ROUTE_BAD_SEQLENS:
            raise ValueError("cu_seqlens were not 0-based, non-decreasing and ending at the token count")


def _check_input(lin: Lin, x: torch.Tensor, what: str) -> None:
    if x.dtype != DT or x.dim() != 2 or x.shape[1] != lin.k or x.stride(1) != 1 or x.device.type != "cuda":
        raise ValueError(f"{', '.join(lin.names)}: {what} takes a bfloat16 (tokens, {lin.k}) input with contiguous "
                         f"rows on the GPU; got {x.dtype} {tuple(x.shape)} with strides {x.stride()}")
    if x.stride(0) % 8 or x.data_ptr() % 16:
        raise ValueError(f"{', '.join(lin.names)}: {what} needs 16-byte aligned input rows")


def lora_add(y: torch.Tensor, x: torch.Tensor, lin: Lin, adp: torch.Tensor, ws: Workspace,
             flags: int = 0) -> torch.Tensor:
    """fast_path.py:277-289, in place: y (M, N) += bf16(x A^T) sB^T with A, sB from the pool row of each token's
    request row (adp, rows of ws.row_len tokens, or the route made by ws.route). One rounding of y + update."""
    _check_input(lin, x, "lora_add")
    m = x.shape[0]
    if y.dtype != DT or y.dim() != 2 or tuple(y.shape) != (m, lin.out) or y.stride(1) != 1:
        raise ValueError(f"lora_add: y must be bfloat16 ({m}, {lin.out}) with contiguous rows")
    if lin.rank > ws.max_rank:
        raise ValueError(f"{', '.join(lin.names)}: stacked rank {lin.rank} exceeds the workspace's {ws.max_rank}")
    r = ws.routed(adp, lin.pool.shape[0], m)
    h = _lib.lib()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    _lib.check(h.mlora_lora_add(lin.lora_abi(), r, x.data_ptr(), x.stride(0), lin.k, y.data_ptr(), y.stride(0),
                                lin.out, ws.mid.data_ptr(), ws.mid.numel() * 2, flags, stream), "mlora_lora_add")
    return y


class AdapterPool:
    """The stacked adapter pool of a set of fused groups (FastPath's lora_pool, fast_path.py:456-547): one bf16 row
    per adapter (row 0: the base), every Lin bound at its offset, and an int32 table of live ranks (one column per
    matrix of every group). Calls must be serialised with the passes that read the pool (as the reference's engine
    thread does)."""

    def __init__(self, lins: Sequence[Lin], max_adapters: int, device: torch.device | str = "cuda") -> None:
        if max_adapters < 1:
            raise ValueError(f"max_adapters={max_adapters}: the fast path needs room for at least one adapter")
        if max_adapters + 1 > _lib.MAX_POOL_ROWS:
            raise ValueError(f"at most {_lib.MAX_POOL_ROWS - 1} adapters")
        self.lins = list(lins)
        self.max_adapters = max_adapters
        self.numel = sum(x.numel() for x in self.lins)
        self.lora_pool = torch.zeros(max_adapters + 1, self.numel, device=device, dtype=DT)
        n_cols = sum(len(x.names) for x in self.lins)
        self.ranks = torch.zeros(max_adapters + 1, max(n_cols, 1), device=device, dtype=torch.int32)
        offset = col = 0
        self.offsets = []
        for x in self.lins:
            x.bind(self.lora_pool, offset, self.ranks, col)
            self.offsets.append(offset)
            offset += x.numel()
            col += len(x.names)
        self.lin_by_name = {name: x for x in self.lins for name in x.names}
        self.adapter_index: dict[str | None, int] = {None: 0}
        self.free_rows = list(range(1, max_adapters + 1))  # sorted: the lowest free row is used first

    def add_adapter(self, name: str, updates: Mapping[str, Update]) -> int:
        """Pack an adapter's updates {matrix name: (A, sB)} into the lowest free row; returns the row
        (fast_path.py:492-522)."""
        if name in self.adapter_index:
            raise ValueError(f"Adapter {name} is already in the fast path")
        if not self.free_rows:
            raise ValueError(f"The fast path holds at most {self.max_adapters} adapters and all "
                             f"{len(self.adapter_index) - 1} are loaded; remove one first")
        unknown = [layer for layer in updates if layer not in self.lin_by_name]
        if unknown:
            raise ValueError(f"Adapter {name} adapts {unknown[0]}, which the fast decision path does not support")
        index = self.free_rows[0]
        row = self.lora_pool[index]
        row.zero_()
        live: list[int] = []
        for x, offset in zip(self.lins, self.offsets):
            live += x.pack(row[offset:offset + x.numel()], {k: v for k, v in updates.items() if k in x.names})
        self.ranks[index, :len(live)] = torch.tensor(live, dtype=torch.int32, device=self.ranks.device)
        self.free_rows.pop(0)
        self.adapter_index[name] = index
        return index

    def remove_adapter(self, name: str, poison: bool = False) -> None:
        """Free the adapter's row (fast_path.py:530-535). Its live ranks become 0, so no kernel reads the row; with
        `poison` the row is filled with NaN, which any read would carry into the outputs."""
        if name is None or name not in self.adapter_index:
            raise ValueError(f"Adapter {name!r} is not loaded in the fast path")
        index = self.adapter_index.pop(name)
        self.ranks[index].zero_()
        if poison:
            self.lora_pool[index].fill_(float("nan"))
        bisect.insort(self.free_rows, index)

    def index(self, adapter: str | None) -> int:
        """The adapter's row in the pool (0: the base) (fast_path.py:542-547)."""
        if adapter not in self.adapter_index:
            raise ValueError(f"Adapter {adapter!r} is not loaded in the fast path")
        return self.adapter_index[adapter]


def attach_int4(lins: Sequence[Lin], quantization) -> int:
    """fast_path.py:352-363: give every Lin of an INT4 base its INT4 weights in the kernel layout from the folder
    `quantization` names (jeff_amd.int4_file.Quantization: its int4.safetensors, checked against the record's
    sha256 and, where the Lin has bfloat16 weights W, against W bit for bit); returns the packed bytes."""
    from jeff_amd.int4_file import attach_int4 as attach
    return attach(lins, quantization)
