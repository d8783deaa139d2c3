"""int4_product: a fused group's INT4 base product plus each token's LoRA update, on the HIP library.

Mirrors the reference's engine/int4_kernels.py:132-177 (int4_product(lin, x, ws, adp, tiles=None)): same arguments,
a new bf16 (tokens, lin.out) result, ValueError before any allocation or launch for a group without INT4 weights, an
input that is not a contiguous bf16 (tokens, lin.k) tensor, or a pass too large for the kernels. On the current
stream: the LoRA first factor, then either the base product with the second factor fused into its epilogue (one
launch, rounded once) or, for passes with few tokens per adapter (decode), the reference's split product: float32
partial products over ranges of the input dimension, then one epilogue launch per (adapter segment, 256 columns)
that adds them in order with the LoRA term and rounds once. Plus the routing launch when the workspace has not
routed `adp` yet. Deterministic: no atomic additions, every sum in a fixed order."""

from __future__ import annotations

import torch

from jeff_amd import _lib
from jeff_amd.fast_path import DT, Lin, Workspace, _check_input
from jeff_amd.int4_tiles import Int4Tiles


EPILOGUES = (None, "silu_mul", "residual")


def _epilogue(lin: Lin, epilogue: str | None) -> tuple[int, int]:
    """(flag bits, output columns) of an epilogue; ValueError for one the group cannot take."""
    if epilogue not in EPILOGUES:
        raise ValueError(f"Unknown epilogue {epilogue!r}; expected one of {EPILOGUES}")
    if epilogue is None:
        return 0, lin.out
    if epilogue == "residual":
        return _lib.EPILOGUE_RESIDUAL, lin.out
    if len(lin.sizes) != 2 or lin.sizes[0] != lin.sizes[1] or lin.sizes[0] % 128 or lin.caps[0] != lin.caps[1] \
            or lin.caps[0] > 64:
        raise ValueError(f"{', '.join(lin.names)}: the silu_mul epilogue takes a gate and an up matrix of one width, a "
                         f"multiple of 128, and one rank capacity of at most 64; got widths {lin.sizes}, capacities "
                         f"{lin.caps}")
    return _lib.EPILOGUE_SILU_MUL, lin.sizes[0]


def _residual_rows(lin: Lin, x: torch.Tensor, residual: torch.Tensor | None, epilogue: str | None,
                   m: int) -> None:
    """ValueError unless `residual` is given exactly for epilogue="residual", as bf16 (m, lin.out) rows that do not
    overlap x (the kernels read x while other tiles write the sums)."""
    if (epilogue == "residual") != (residual is not None):
        raise ValueError("epilogue='residual' takes the residual rows (residual=...), and no other epilogue does")
    if residual is None:
        return
    if residual.dtype != DT or residual.dim() != 2 or tuple(residual.shape) != (m, lin.out) or \
            residual.stride(1) != 1 or residual.device != x.device:
        raise ValueError(f"residual must be a bfloat16 ({m}, {lin.out}) tensor with contiguous rows on {x.device}")

    def span(t: torch.Tensor) -> tuple[int, int]:
        return t.data_ptr(), t.data_ptr() + ((t.shape[0] - 1) * t.stride(0) + t.shape[1]) * t.element_size()

    (a0, a1), (b0, b1) = span(x), span(residual)
    if a0 < b1 and b0 < a1:
        raise ValueError("residual must not overlap x")


def int4_product(lin: Lin, x: torch.Tensor, ws: Workspace, adp: torch.Tensor, tiles: Int4Tiles | None = None,
                 last_out: torch.Tensor | None = None, epilogue: str | None = None,
                 residual: torch.Tensor | None = None) -> torch.Tensor:
    """The fused product of x (M, in) through `lin`'s INT4 weights plus each token's adapter update (the pool row of
    its request row in adp, or the route ws.route made). `tiles` forces the kernel families (tests); `last_out`
    (requests, columns) bf16 also receives each request's last-token output row. epilogue="silu_mul" (a gate_up
    group: gate then up, one width each): the result is silu_mul of the product, (M, width) (the reference's
    silu_mul(product(...)), engine/batched_path.py:271, in the product's own output tile, bit for bit).
    epilogue="residual" with residual=r, (M, out) bf16: the residual add of add_rms in the output tile, r updated in
    place to bf16(r + product) and returned (the x of the reference's add_rms(x, product(...), w),
    engine/fast_path.py:80-100, bit for bit; the last-token rows receive the sums)."""
    packed = lin.int4
    if packed is None:
        raise ValueError(f"{', '.join(lin.names)}: no INT4 weights (attach_int4 gives them to an INT4 base's fused "
                         "groups only)")
    eflag, cols = _epilogue(lin, epilogue)
    _check_input(lin, x, "the INT4 product")
    m = x.shape[0]
    if m >= 2 ** 31 - 1:
        raise ValueError(f"{', '.join(lin.names)}: {m} tokens reach 2^31; the kernels' token offsets are 32-bit")
    if tiles is not None and tiles.base == "gemv" and m > 8:
        raise ValueError(f"the GEMV base product runs at most 8 tokens; got {m}")
    if lin.rank > ws.max_rank:
        raise ValueError(f"{', '.join(lin.names)}: stacked rank {lin.rank} exceeds the workspace's {ws.max_rank}")
    if last_out is not None and (last_out.dtype != DT or last_out.dim() != 2 or last_out.shape[1] != cols
                                 or not last_out.is_contiguous() or last_out.shape[0] < adp.numel()):
        raise ValueError(f"last_out must be a contiguous bfloat16 (requests, {cols}) tensor")
    _residual_rows(lin, x, residual, epilogue, m)
    r = ws.routed(adp, lin.pool.shape[0], m)
    y = residual if residual is not None else torch.empty(m, cols, device=x.device, dtype=DT)
    h = _lib.lib()
    flags = (0 if tiles is None else tiles.flags()) | eflag
    w, lora = packed.abi(), lin.lora_abi()
    part, part_bytes = ws.partials(h.mlora_int4_partials_bytes(w, lora, r, flags))
    stream = torch.cuda.current_stream(x.device).cuda_stream
    _lib.check(h.mlora_int4_linear(w, lora, r, x.data_ptr(), x.stride(0), y.data_ptr(), y.stride(0),
                                   0 if last_out is None else last_out.data_ptr(), ws.mid.data_ptr(),
                                   ws.mid.numel() * 2, part, part_bytes, flags, stream),
               "mlora_int4_linear")
    return y


def shrink(lin: Lin, x: torch.Tensor, ws: Workspace, adp: torch.Tensor, mfma: bool | None = None) -> torch.Tensor:
    """The LoRA first factors the products use, at sorted token positions: a (tokens, lin.rank) bf16 view of the
    workspace, matrix j's live ranks in columns [rho_j, rho_j + rank) (other columns are left as they were)."""
    _check_input(lin, x, "shrink")
    m = x.shape[0]
    r = ws.routed(adp, lin.pool.shape[0], m)
    flags = 0 if mfma is None else (_lib.FORCE_SHRINK_MFMA if mfma else _lib.FORCE_SHRINK_SEGMENT)
    h = _lib.lib()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    _lib.check(h.mlora_shrink(lin.lora_abi(), r, x.data_ptr(), x.stride(0), lin.k, ws.mid.data_ptr(), flags, stream),
               "mlora_shrink")
    return ws.mid[:m * lin.rank].view(m, lin.rank)


def base_expand(lin: Lin, x: torch.Tensor, ws: Workspace, adp: torch.Tensor, y: torch.Tensor,
                tiles: Int4Tiles | None = None, last_out: torch.Tensor | None = None,
                epilogue: str | None = None) -> torch.Tensor:
    """int4_product without its first launch, into a given y: the base product and the LoRA second factor, reading
    the first factors the last shrink (or int4_product) of the same x and adp left in the workspace. With
    epilogue="residual", y holds the residual rows and receives the sums."""
    packed = lin.int4
    if packed is None:
        raise ValueError(f"{', '.join(lin.names)}: no INT4 weights")
    eflag, cols = _epilogue(lin, epilogue)
    _check_input(lin, x, "the INT4 product")
    m = x.shape[0]
    if y.dtype != DT or tuple(y.shape) != (m, cols) or y.stride(1) != 1:
        raise ValueError(f"y must be bfloat16 ({m}, {cols}) with contiguous rows")
    if epilogue == "residual":
        _residual_rows(lin, x, y, epilogue, m)
    r = ws.routed(adp, lin.pool.shape[0], m)
    h = _lib.lib()
    flags = (0 if tiles is None else tiles.flags()) | eflag
    w, lora = packed.abi(), lin.lora_abi()
    part, part_bytes = ws.partials(h.mlora_int4_partials_bytes(w, lora, r, flags))
    stream = torch.cuda.current_stream(x.device).cuda_stream
    _lib.check(h.mlora_int4_base_expand(w, lora, r, x.data_ptr(), x.stride(0), y.data_ptr(), y.stride(0),
                                        0 if last_out is None else last_out.data_ptr(), ws.mid.data_ptr(), part,
                                        part_bytes, flags, stream),
               "mlora_int4_base_expand")
    return y
