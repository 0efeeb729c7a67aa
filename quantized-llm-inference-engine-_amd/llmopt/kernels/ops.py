"""Torch-facing wrappers over the C ABI of ``libllmopt_qlinear.so``.

These are the only entry points the quantization layer uses on HIP devices:

* :func:`unpack_nibbles` replaces ``unpack_int4`` (``quantizers.py:92-97``),
* :func:`dequantize` replaces ``dequantize`` (``quantizers.py:231-239``),
* :func:`quant_linear` replaces the dequantize-then-``F.linear`` body of
  ``QuantLinear.forward`` (``quant_linear.py:93-113``),
* :func:`quantize_rtn` replaces ``RoundToNearestQuantizer.quantize``
  (``quantizers.py:285-305``) in one pass over the weight,
* :func:`kv_write_decode` / :func:`kv_write` replace ``PagedKVCache.write_decode`` / ``write``
  (``src/llmopt/cache/paged_cache.py:187-277``),
* :func:`paged_decode_attention` replaces ``PagedAttention.forward`` for one query token per
  sequence (``src/llmopt/attention/paged_attention.py:145-290``), reading the cache in place.

Each wrapper checks what torch would check (dtypes, devices, shapes), passes raw
device pointers and the current HIP stream to the library, and raises if the
library is missing or reports an error. Nothing here computes on the host.
"""

from __future__ import annotations

import ctypes

import torch

from llmopt.kernels._lib import ALGO_AUTO, ALGO_DENSE, DTYPE_CODES, call, load_library

__all__ = [
    "dequantize",
    "kv_write",
    "kv_write_decode",
    "paged_decode_attention",
    "quant_linear",
    "quant_linear_swiglu",
    "quantize_rtn",
    "rmsnorm",
    "rmsnorm_supported",
    "rope",
    "rope_kv_write_decode",
    "paged_decode_attention_rope",
    "argmax_rows",
    "paged_prefill_attention",
    "unpack_nibbles",
]


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _same_device(x: torch.Tensor, *others: torch.Tensor | None) -> None:
    for other in others:
        if other is not None and other.device != x.device:
            raise RuntimeError(
                "Expected all tensors to be on the same device, but found at least two devices, "
                f"{x.device} and {other.device}!"
            )


def _metadata(tensor: torch.Tensor, rows: int, groups: int, what: str) -> torch.Tensor:
    """fp32 contiguous ``[rows, groups]`` view of scales/zeros, broadcasting like torch."""
    if tensor.dtype != torch.float32:
        tensor = tensor.to(torch.float32)
    if tuple(tensor.shape) != (rows, groups):
        try:
            tensor = tensor.expand(rows, groups)
        except RuntimeError as exc:
            raise RuntimeError(
                f"{what} of shape {tuple(tensor.shape)} does not broadcast to ({rows}, {groups})"
            ) from exc
    return tensor.contiguous()


def _weight_args(qt, device: torch.device):  # noqa: ANN001, ANN202 - QuantizedTensor
    """Validated (qweight, ldq, scales, zeros, N, K, group, signed) for a QuantizedTensor."""
    rows, cols = (int(d) for d in qt.shape)
    bits = int(qt.bits)
    if not 1 <= bits <= 8:
        raise ValueError(f"unsupported bit width: {bits}")
    group = cols if qt.group_size is None or qt.group_size <= 0 else int(qt.group_size)
    if cols % group:
        raise RuntimeError(
            f"shape '[{rows}, {cols // group}, {group}]' is invalid for input of size {rows * cols}"
        )
    qweight = qt.qweight
    _same_device(qweight, qt.scales, None if qt.symmetric else qt.zeros)
    if qweight.device != device:
        _same_device(torch.empty(0, device=device), qweight)
    if bits < 8 and qweight.dtype != torch.uint8:
        raise TypeError(f"{bits}-bit codes must be packed as uint8, got {qweight.dtype}")
    if bits == 8 and qweight.dtype not in (torch.uint8, torch.int8):
        raise TypeError(f"8-bit codes must be uint8 or int8, got {qweight.dtype}")
    qweight = qweight.contiguous()
    if qweight.dim() != 2 or qweight.shape[0] != rows:
        raise RuntimeError(f"qweight of shape {tuple(qweight.shape)} does not match weight {rows}x{cols}")
    needed = cols if bits == 8 else (cols + 1) // 2
    if qweight.shape[1] < needed:
        raise RuntimeError(
            f"qweight row of {qweight.shape[1]} bytes cannot hold {cols} {bits}-bit codes"
        )
    groups = cols // group if cols else 0
    scales = _metadata(qt.scales, rows, groups, "scales")
    zeros = None if qt.symmetric else _metadata(qt.zeros, rows, groups, "zeros")
    signed = qweight.dtype == torch.int8
    return qweight, int(qweight.shape[1]), scales, zeros, rows, cols, int(qt.group_size), signed


def quantize_rtn(
    weight: torch.Tensor, bits: int, group_size: int, symmetric: bool
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Round-to-nearest quantization of a HIP weight ``[out, in]``: ``(qweight, scales, zeros)``.

    Bit-exact with ``choose_qparams`` + ``quantize_to_codes`` + ``pack_int4`` on the host
    (``quantizers.py:83-89,100-142,167-201``): ``qweight`` is ``uint8 [out, in/2]`` below 8 bits,
    ``uint8``/``int8 [out, in]`` at 8 bits (asymmetric/symmetric); ``scales`` and ``zeros`` are
    fp32 ``[out, in/group]`` (``zeros`` all 0 when symmetric). float64 weights are rounded to
    fp32 first, which commutes with the reference's min/max and is what its division sees.
    """
    if weight.dim() != 2:
        raise ValueError(f"expected a 2D weight, got shape {tuple(weight.shape)}")
    if not weight.is_floating_point():
        raise TypeError(f"expected a floating-point weight, got {weight.dtype}")
    if weight.dtype == torch.float64:
        weight = weight.to(torch.float32)
    rows, cols = (int(d) for d in weight.shape)
    group = cols if group_size is None or group_size <= 0 else int(group_size)
    if cols % group:
        raise ValueError(f"in_features={cols} not divisible by group_size={group}")
    w = weight.contiguous()
    dev = w.device
    if bits == 8:
        qweight = torch.empty(rows, cols, dtype=torch.int8 if symmetric else torch.uint8, device=dev)
    else:
        qweight = torch.empty(rows, cols // 2, dtype=torch.uint8, device=dev)
    groups = cols // group if cols else 0
    scales = torch.empty(rows, groups, dtype=torch.float32, device=dev)
    zeros = torch.empty(rows, groups, dtype=torch.float32, device=dev)
    lib = load_library()
    call(
        lib.llmopt_q_quantize_rtn(
            w.data_ptr(), DTYPE_CODES[w.dtype], cols, rows, cols, int(bits), group, int(bool(symmetric)),
            qweight.data_ptr(), int(qweight.shape[1]), scales.data_ptr(), zeros.data_ptr(),
            _stream_handle(dev),
        ),
        "llmopt_q_quantize_rtn",
    )
    return qweight, scales, zeros


def unpack_nibbles(packed: torch.Tensor, columns: int) -> torch.Tensor:
    """``unpack_int4`` on a HIP tensor: ``[..., P]`` uint8 -> ``[..., min(columns, 2P)]``."""
    if packed.dtype != torch.uint8:
        raise TypeError(f"packed nibbles must be uint8, got {packed.dtype}")
    packed = packed.contiguous()
    width = packed.shape[-1] if packed.dim() else 1
    keep = len(range(2 * width)[:columns])
    out = torch.empty(*packed.shape[:-1], keep, dtype=torch.uint8, device=packed.device)
    rows = packed.numel() // width if width else 0
    if out.numel() == 0:
        return out
    lib = load_library()
    call(
        lib.llmopt_q_unpack(
            packed.data_ptr(), out.data_ptr(), rows, width, keep, _stream_handle(packed.device)
        ),
        "llmopt_q_unpack",
    )
    return out


def dequantize(qt, dtype: torch.dtype = torch.float32) -> torch.Tensor:  # noqa: ANN001
    """Dense ``[N, K]`` weight from a QuantizedTensor whose tensors live on a HIP device.

    The kernel evaluates the reference's fp32 ``(q - z) * s`` bit for bit and casts to
    fp32, fp16 or bf16 with round-to-nearest-even; other dtypes are produced from the
    fp32 result with ``.to(dtype)``, the same final step the reference takes.
    """
    device = qt.qweight.device
    qweight, ldq, scales, zeros, rows, cols, group, signed = _weight_args(qt, device)
    native = dtype if dtype in DTYPE_CODES else torch.float32
    out = torch.empty(rows, cols, dtype=native, device=device)
    if out.numel():
        lib = load_library()
        call(
            lib.llmopt_q_dequant(
                qweight.data_ptr(),
                ldq,
                scales.data_ptr(),
                zeros.data_ptr() if zeros is not None else None,
                out.data_ptr(),
                DTYPE_CODES[native],
                rows,
                cols,
                int(qt.bits),
                group,
                int(bool(qt.symmetric)),
                int(signed),
                _stream_handle(device),
            ),
            "llmopt_q_dequant",
        )
    return out if native == dtype else out.to(dtype)


class PartialSums:
    """A linear's output left as the K-split partial sums of its decode kernel: ``planes``
    ``[S, M, N]`` fp32 (the bias not added), ``bias`` (``[N]`` or None), the output ``dtype`` and
    ``shape``. :func:`rmsnorm` with a residual adds them up inside its kernel;
    :meth:`materialize` gives the output tensor, as the split-K reduction computes it."""

    def __init__(self, planes: torch.Tensor, bias: torch.Tensor | None, dtype: torch.dtype,
                 shape: tuple[int, ...]) -> None:
        self.planes = planes
        self.bias = bias
        self.dtype = dtype
        self.shape = torch.Size(shape)
        self.device = planes.device

    def materialize(self) -> torch.Tensor:
        """The slices added in order, then the bias, rounded once: the reduction's arithmetic."""
        v = self.planes[0]
        for s in range(1, int(self.planes.shape[0])):
            v = v + self.planes[s]
        if self.bias is not None:
            v = v + self.bias.float()
        return v.to(self.dtype).view(self.shape)


def quant_linear(
    x: torch.Tensor,
    qt,  # noqa: ANN001 - QuantizedTensor
    bias: torch.Tensor | None,
    compute_dtype: torch.dtype,
    algo: int = ALGO_AUTO,
    defer: bool = False,
) -> torch.Tensor | PartialSums:
    """``F.linear(x, dequantize(qt, compute_dtype), bias)`` without a dense weight.

    Raises the errors ``F.linear`` would raise for mismatched dtypes, devices or shapes. With
    ``defer`` (16-bit activations), a batch whose plan is the K-sliced decode kernel returns
    its :class:`PartialSums` instead of the output (``llmopt_q_linear_deferred``).
    """
    if x.dtype != compute_dtype:
        raise RuntimeError(
            f"expected m1 and m2 to have the same dtype, but got: {x.dtype} != {compute_dtype}"
        )
    if compute_dtype not in DTYPE_CODES:
        raise TypeError(f"compute_dtype {compute_dtype} is not supported by the HIP kernels")
    if bias is not None and bias.dtype != compute_dtype:
        raise RuntimeError(
            f"self and mat2 must have the same dtype, but got {bias.dtype} and {compute_dtype}"
        )
    _same_device(x, qt.qweight, qt.scales, bias)
    qweight, ldq, scales, zeros, rows, cols, group, signed = _weight_args(qt, x.device)
    if x.dim() == 0 or x.shape[-1] != cols:
        lead = x.numel() // x.shape[-1] if x.dim() and x.shape[-1] else 0
        raise RuntimeError(
            f"mat1 and mat2 shapes cannot be multiplied ({lead}x{x.shape[-1] if x.dim() else 0} "
            f"and {cols}x{rows})"
        )
    lead_shape = x.shape[:-1]
    x2 = x.reshape(-1, cols)
    if cols and x2.stride(-1) != 1:
        x2 = x2.contiguous()
    m = x2.shape[0]
    ldx = x2.stride(0) if m > 1 else cols
    y = torch.empty(m, rows, dtype=compute_dtype, device=x.device)
    if m and rows:
        if bias is not None:
            bias = bias.contiguous()
        lib = load_library()
        # Scratch for split-K partial sums, or from 1024 tokens (65 in fp32) the dense weight of
        # the two-pass path; it comes from torch's caching allocator, so repeated calls reuse
        # the same block.
        if algo == ALGO_DENSE:
            ws_bytes = int(lib.llmopt_q_linear_dense_workspace(rows, cols, DTYPE_CODES[compute_dtype]))
        else:
            ws_bytes = int(
                lib.llmopt_q_linear_workspace_ex(m, rows, cols, int(qt.bits), group, DTYPE_CODES[compute_dtype])
            )
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
        if defer and algo == ALGO_AUTO and compute_dtype != torch.float32:
            planes = ctypes.c_int(0)
            call(
                lib.llmopt_q_linear_deferred(
                    x2.data_ptr(), m, cols, max(ldx, cols), qweight.data_ptr(), ldq, scales.data_ptr(),
                    zeros.data_ptr() if zeros is not None else None, bias.data_ptr() if bias is not None else None,
                    y.data_ptr(), rows, rows, DTYPE_CODES[compute_dtype], int(qt.bits), group,
                    int(bool(qt.symmetric)), int(signed), ws.data_ptr() if ws is not None else None, ws_bytes,
                    _stream_handle(x.device), ctypes.byref(planes),
                ),
                "llmopt_q_linear_deferred",
            )
            if planes.value:
                s = int(planes.value)
                pl = ws[: s * m * rows * 4].view(torch.float32).view(s, m, rows)
                return PartialSums(pl, bias, compute_dtype, (*lead_shape, rows))
            return y.reshape(*lead_shape, rows)
        call(
            lib.llmopt_q_linear_ex(
                x2.data_ptr(),
                m,
                cols,
                max(ldx, cols),
                qweight.data_ptr(),
                ldq,
                scales.data_ptr(),
                zeros.data_ptr() if zeros is not None else None,
                bias.data_ptr() if bias is not None else None,
                y.data_ptr(),
                rows,
                rows,
                DTYPE_CODES[compute_dtype],
                int(qt.bits),
                group,
                int(bool(qt.symmetric)),
                int(signed),
                ws.data_ptr() if ws is not None else None,
                ws_bytes,
                _stream_handle(x.device),
                int(algo),
            ),
            "llmopt_q_linear",
        )
    return y.reshape(*lead_shape, rows)


ERR_WORKSPACE = -4


def quant_linear_swiglu(
    x: torch.Tensor,
    qt,  # noqa: ANN001 - QuantizedTensor with gate and up rows interleaved in blocks of four
    bias: torch.Tensor | None,
    compute_dtype: torch.dtype,
) -> torch.Tensor:
    """``silu(x @ gate^T) * (x @ up^T)`` from one fused weight, without the [M, 2I] product.

    ``qt`` holds ``2I`` rows: fused row ``8p + r`` is gate row ``4p + r`` and ``8p + 4 + r`` is
    up row ``4p + r`` (``r < 4``); ``bias`` (if any) follows the same order. Returns ``[..., I]``.
    """
    if x.dtype != compute_dtype:
        raise RuntimeError(
            f"expected m1 and m2 to have the same dtype, but got: {x.dtype} != {compute_dtype}"
        )
    if compute_dtype not in DTYPE_CODES:
        raise TypeError(f"compute_dtype {compute_dtype} is not supported by the HIP kernels")
    if bias is not None and bias.dtype != compute_dtype:
        raise RuntimeError(
            f"self and mat2 must have the same dtype, but got {bias.dtype} and {compute_dtype}"
        )
    _same_device(x, qt.qweight, qt.scales, bias)
    qweight, ldq, scales, zeros, rows, cols, group, signed = _weight_args(qt, x.device)
    if rows % 8:
        raise ValueError(f"fused gate/up weight needs a multiple of 8 rows, got {rows}")
    if x.dim() == 0 or x.shape[-1] != cols:
        lead = x.numel() // x.shape[-1] if x.dim() and x.shape[-1] else 0
        raise RuntimeError(
            f"mat1 and mat2 shapes cannot be multiplied ({lead}x{x.shape[-1] if x.dim() else 0} "
            f"and {cols}x{rows})"
        )
    lead_shape = x.shape[:-1]
    x2 = x.reshape(-1, cols)
    if cols and x2.stride(-1) != 1:
        x2 = x2.contiguous()
    m = x2.shape[0]
    ldx = x2.stride(0) if m > 1 else cols
    out = rows // 2
    y = torch.empty(m, out, dtype=compute_dtype, device=x.device)
    if m and rows:
        if bias is not None:
            bias = bias.contiguous()
        lib = load_library()
        ws_bytes = int(
            lib.llmopt_q_linear_swiglu_workspace_ex(m, rows, cols, int(qt.bits), group, DTYPE_CODES[compute_dtype])
        )
        for _attempt in range(2):
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
            rc = lib.llmopt_q_linear_swiglu(
                x2.data_ptr(), m, cols, max(ldx, cols), qweight.data_ptr(), ldq, scales.data_ptr(),
                zeros.data_ptr() if zeros is not None else None,
                bias.data_ptr() if bias is not None else None,
                y.data_ptr(), rows, out, DTYPE_CODES[compute_dtype], int(qt.bits), group,
                int(bool(qt.symmetric)), int(signed), ws.data_ptr() if ws is not None else None,
                ws_bytes, _stream_handle(x.device),
            )
            if rc != ERR_WORKSPACE:
                break
            # A kernel without the fused activation ran into a short workspace (an unusual
            # alignment): give it room for the full product and try once more.
            ws_bytes = (m * rows * 4 + 255) // 256 * 256 + int(
                lib.llmopt_q_linear_workspace_ex(m, rows, cols, int(qt.bits), group, DTYPE_CODES[compute_dtype])
            )
        call(rc, "llmopt_q_linear_swiglu")
    return y.reshape(*lead_shape, out)


# ---- paged KV cache and decode attention -------------------------------------------------------

def _int32(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    return t.to(device=device, dtype=torch.int32).contiguous()


def _check_rows(what: str, seqs: int, **tensors: torch.Tensor) -> None:
    """Each per-sequence tensor must have a row for every one of ``seqs`` sequences: the
    kernels read row ``s`` of each for every ``s < seqs`` (the reference's indexing raises)."""
    for name, t in tensors.items():
        rows = int(t.shape[0]) if t.dim() > 0 else 1
        if rows < seqs:
            raise ValueError(f"{what}: {name} has {rows} rows for {seqs} sequences")


def _layer_cache(key_cache: torch.Tensor, value_cache: torch.Tensor) -> tuple[int, int, int, int, int]:
    """Geometry of one layer's caches ``[num_blocks, block_size, kv_heads, head_dim]``."""
    if key_cache.dim() != 4 or key_cache.shape != value_cache.shape:
        raise ValueError(f"expected two [blocks, block_size, kv_heads, head_dim] caches, got "
                         f"{tuple(key_cache.shape)} and {tuple(value_cache.shape)}")
    if key_cache.dtype != value_cache.dtype or key_cache.dtype not in DTYPE_CODES:
        raise TypeError(f"unsupported cache dtypes {key_cache.dtype}, {value_cache.dtype}")
    if not (key_cache.is_contiguous() and value_cache.is_contiguous()):
        raise ValueError("the caches must be contiguous")
    nb, bs, kvh, hd = (int(d) for d in key_cache.shape)
    return nb, bs, kvh, hd, DTYPE_CODES[key_cache.dtype]


def kv_write_decode(key_cache, value_cache, block_ids, token_offsets, keys, values) -> None:  # noqa: ANN001
    """``PagedKVCache.write_decode`` for one layer: ``keys``/``values`` ``[seq, kv_heads, head_dim]``."""
    nb, bs, kvh, hd, cdt = _layer_cache(key_cache, value_cache)
    seqs = int(keys.shape[0])
    if seqs == 0:
        return
    dev = key_cache.device
    if keys.dtype not in DTYPE_CODES:
        keys, values = keys.to(key_cache.dtype), values.to(key_cache.dtype)
    if int(values.shape[0]) != seqs or block_ids.dim() != 2:
        raise ValueError("kv_write_decode: values must match keys, block_ids must be [seqs, blocks]")
    _check_rows("kv_write_decode", seqs, block_ids=block_ids, token_offsets=token_offsets.reshape(-1))
    k = keys.reshape(seqs, kvh * hd).contiguous()
    v = values.reshape(seqs, kvh * hd).to(k.dtype).contiguous()
    table = _int32(block_ids, dev)
    offsets = _int32(token_offsets, dev)
    lib = load_library()
    call(
        lib.llmopt_kv_write_decode(
            key_cache.data_ptr(), value_cache.data_ptr(), cdt, nb, bs, kvh, hd, table.data_ptr(),
            int(table.shape[1]), offsets.data_ptr(), k.data_ptr(), v.data_ptr(), DTYPE_CODES[k.dtype],
            kvh * hd, seqs, _stream_handle(dev),
        ),
        "llmopt_kv_write_decode",
    )


def kv_write(key_cache, value_cache, block_ids, token_offsets, keys, values) -> None:  # noqa: ANN001
    """``PagedKVCache.write`` for one layer: ``keys``/``values`` ``[seq, q_len, kv_heads, head_dim]``."""
    nb, bs, kvh, hd, cdt = _layer_cache(key_cache, value_cache)
    seqs, q_len = int(keys.shape[0]), int(keys.shape[1])
    if seqs == 0 or q_len == 0:
        return
    dev = key_cache.device
    if keys.dtype not in DTYPE_CODES:
        keys, values = keys.to(key_cache.dtype), values.to(key_cache.dtype)
    if int(values.shape[0]) != seqs or block_ids.dim() != 2:
        raise ValueError("kv_write: values must match keys, block_ids must be [seqs, blocks]")
    _check_rows("kv_write", seqs, block_ids=block_ids, token_offsets=token_offsets.reshape(-1))
    k = keys.reshape(seqs, q_len, kvh * hd).contiguous()
    v = values.reshape(seqs, q_len, kvh * hd).to(k.dtype).contiguous()
    table = _int32(block_ids, dev)
    offsets = _int32(token_offsets, dev)
    lib = load_library()
    call(
        lib.llmopt_kv_write(
            key_cache.data_ptr(), value_cache.data_ptr(), cdt, nb, bs, kvh, hd, table.data_ptr(),
            int(table.shape[1]), offsets.data_ptr(), k.data_ptr(), v.data_ptr(), DTYPE_CODES[k.dtype],
            q_len * kvh * hd, kvh * hd, seqs, q_len, _stream_handle(dev),
        ),
        "llmopt_kv_write",
    )


def paged_decode_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_ids: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    softcap: float = 0.0,
) -> torch.Tensor:
    """Decode attention for ``query [seq, heads, head_dim]`` over one layer's paged caches.

    Returns ``[seq, heads, head_dim]`` in the query's dtype. Raises ``NotImplementedError`` for
    shapes the kernel does not take (fp32 caches, head_dim other than 64/128, more than 16 or a
    non-power-of-two number of query heads per KV head).
    """
    nb, bs, kvh, hd, cdt = _layer_cache(key_cache, value_cache)
    if query.dim() != 3 or int(query.shape[2]) != hd:
        raise ValueError(f"query of shape {tuple(query.shape)} does not match head_dim {hd}")
    if query.dtype not in DTYPE_CODES:
        raise TypeError(f"unsupported query dtype {query.dtype}")
    seqs, heads = int(query.shape[0]), int(query.shape[1])
    dev = key_cache.device
    q = query.contiguous()
    out = torch.empty(seqs, heads, hd, dtype=query.dtype, device=dev)
    if seqs == 0:
        return out
    table = _int32(block_ids, dev)
    lens = _int32(context_lens, dev)
    ldb = int(table.shape[1])
    lib = load_library()
    ws_bytes = lib.llmopt_paged_attention_workspace(seqs, heads, kvh, hd, ldb, bs)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    call(
        lib.llmopt_paged_attention_decode(
            q.data_ptr(), DTYPE_CODES[q.dtype], heads * hd, key_cache.data_ptr(), value_cache.data_ptr(), cdt,
            nb, bs, kvh, hd, table.data_ptr(), ldb, lens.data_ptr(), seqs, heads, float(scale), float(softcap),
            out.data_ptr(), None if ws is None else ws.data_ptr(), ws_bytes, _stream_handle(dev),
        ),
        "llmopt_paged_attention_decode",
    )
    return out



def paged_prefill_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_ids: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    softcap: float = 0.0,
) -> torch.Tensor:
    """Prefill attention for ``query [seq, heads, q_len, head_dim]`` (any strides with a unit
    inner stride) over one layer's paged caches, this step's K/V already written: query token j
    sits at ``context_lens - q_len + j`` and sees the keys up to its own position. Returns
    ``[seq, heads, q_len, head_dim]`` in the query's dtype -- a view of a ``[seq, q_len, heads,
    head_dim]`` buffer, the layout the output projection reads. Raises ``NotImplementedError``
    for shapes the kernel does not take (as :func:`paged_decode_attention`)."""
    nb, bs, kvh, hd, cdt = _layer_cache(key_cache, value_cache)
    if query.dim() != 4 or int(query.shape[3]) != hd:
        raise ValueError(f"query of shape {tuple(query.shape)} does not match head_dim {hd}")
    if query.dtype not in DTYPE_CODES:
        raise TypeError(f"unsupported query dtype {query.dtype}")
    seqs, heads, q_len = (int(d) for d in query.shape[:3])
    dev = key_cache.device
    q = query if query.stride(3) == 1 else query.contiguous()
    out = torch.empty(seqs, q_len, heads, hd, dtype=query.dtype, device=dev)
    view = out.permute(0, 2, 1, 3)
    if seqs == 0 or q_len == 0:
        return view
    _check_rows("paged_prefill_attention", seqs, block_ids=block_ids, context_lens=context_lens.reshape(-1))
    table = _int32(block_ids, dev)
    lens = _int32(context_lens, dev)
    call(
        load_library().llmopt_paged_attention_prefill(
            q.data_ptr(), DTYPE_CODES[q.dtype], q.stride(0), q.stride(2), q.stride(1), key_cache.data_ptr(),
            value_cache.data_ptr(), cdt, nb, bs, kvh, hd, table.data_ptr(), int(table.shape[1]), lens.data_ptr(),
            seqs, heads, q_len, float(scale), float(softcap), out.data_ptr(), q_len * heads * hd, heads * hd, hd,
            _stream_handle(dev),
        ),
        "llmopt_paged_attention_prefill",
    )
    return view


def paged_decode_attention_rope(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    positions: torch.Tensor,
    cos_table: torch.Tensor,
    sin_table: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_ids: torch.Tensor,
    context_lens: torch.Tensor,
    token_offsets: torch.Tensor,
    scale: float,
    softcap: float = 0.0,
) -> torch.Tensor:
    """The attention layer's decode step in one launch: :func:`rope_kv_write_decode` (rotate q
    and k, store k and v at ``token_offsets``) then :func:`paged_decode_attention`, with the same
    results. ``q [seqs, heads, d]`` and ``k``/``v [seqs, kv_heads, d]`` are the raw projection
    rows (unit inner strides), in the cache dtype (bf16 or fp16); returns ``[seqs, heads, d]``.
    Raises ``NotImplementedError`` where either kernel would (see :func:`paged_decode_attention`).
    The slot a sequence writes must not be a key of another sequence in the same call."""
    seqs, heads, d = (int(s) for s in q.shape)
    kv_heads = int(k.shape[1])
    nb, bs, kvh, hd, cdt = _layer_cache(key_cache, value_cache)
    if q.dtype != key_cache.dtype or k.dtype != q.dtype or v.dtype != q.dtype or (kvh, hd) != (kv_heads, d) \
            or tuple(v.shape) != tuple(k.shape):
        raise ValueError("paged_decode_attention_rope: cache dtype/shape does not match q/k/v")
    if int(k.shape[0]) != seqs or block_ids.dim() != 2:
        raise ValueError("paged_decode_attention_rope: k/v need one row per query row, block_ids [seqs, blocks]")
    _check_rows("paged_decode_attention_rope", seqs, positions=positions.reshape(-1),
                token_offsets=token_offsets.reshape(-1), block_ids=block_ids, context_lens=context_lens.reshape(-1))

    def inner_ok(t: torch.Tensor) -> bool:
        return t.stride(2) == 1 and t.stride(1) == d

    q, k, v = (t if inner_ok(t) else t.contiguous() for t in (q, k, v))
    dev = key_cache.device
    out = torch.empty(seqs, heads, d, dtype=q.dtype, device=dev)
    if seqs == 0:
        return out
    pos = positions.to(device=dev, dtype=torch.int64).contiguous()
    cos_t = cos_table.to(device=dev, dtype=torch.float32).contiguous()
    sin_t = sin_table.to(device=dev, dtype=torch.float32).contiguous()
    table = _int32(block_ids, dev)
    offsets = _int32(token_offsets, dev)
    lens = _int32(context_lens, dev)
    ldb = int(table.shape[1])
    lib = load_library()
    ws_bytes = lib.llmopt_paged_attention_workspace(seqs, heads, kvh, hd, ldb, bs)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    call(
        lib.llmopt_paged_attention_decode_rope(
            q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0), pos.data_ptr(),
            cos_t.data_ptr(), sin_t.data_ptr(), int(cos_t.shape[0]), cdt, key_cache.data_ptr(),
            value_cache.data_ptr(), nb, bs, kvh, hd, table.data_ptr(), ldb, offsets.data_ptr(), lens.data_ptr(),
            seqs, heads, float(scale), float(softcap), out.data_ptr(), None if ws is None else ws.data_ptr(),
            ws_bytes, _stream_handle(dev),
        ),
        "llmopt_paged_attention_decode_rope",
    )
    return out


def argmax_rows(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``torch.argmax(x, dim=-1)`` of a 2-D device tensor (fp32 / fp16 / bf16, unit inner
    stride) as one kernel: the first maximum of each row, NaN above every number; int64
    ``[rows]``, written into ``out`` when given (contiguous int64 ``[rows]`` on the same device).
    The greedy sampler's step (``sampler.py:94-95``)."""
    if x.dim() != 2 or x.dtype not in DTYPE_CODES:
        raise ValueError(f"argmax_rows takes a 2-D fp32/fp16/bf16 tensor, got {tuple(x.shape)} {x.dtype}")
    if x.stride(1) != 1:
        x = x.contiguous()
    rows, cols = (int(d) for d in x.shape)
    if out is None:
        out = torch.empty(rows, dtype=torch.long, device=x.device)
    elif (out.dtype != torch.long or tuple(out.shape) != (rows,) or not out.is_contiguous()
          or out.device != x.device):
        raise ValueError(f"out must be a contiguous int64 [{rows}] tensor on {x.device}")
    if rows == 0:
        return out
    if cols == 0:
        raise ValueError("argmax_rows of an empty row")
    call(
        load_library().llmopt_argmax_rows(x.data_ptr(), DTYPE_CODES[x.dtype], rows, cols, max(x.stride(0), cols),
                                          out.data_ptr(), _stream_handle(x.device)),
        "llmopt_argmax_rows",
    )
    return out


# ---- decoder elementwise steps -------------------------------------------------------------------


def rmsnorm_supported(x: torch.Tensor | PartialSums, weight: torch.Tensor,
                      residual: torch.Tensor | None = None) -> bool:
    """Whether :func:`rmsnorm` takes these tensors (bf16/fp16 on a HIP device, 16-byte rows;
    :class:`PartialSums` with a residual)."""
    if isinstance(x, PartialSums):
        return (residual is not None and residual.shape == x.shape and residual.dtype == x.dtype
                and x.dtype in (torch.bfloat16, torch.float16) and weight.dtype == x.dtype
                and int(x.shape[-1]) % 8 == 0 and weight.numel() == int(x.shape[-1]) and weight.is_contiguous()
                and residual.is_contiguous() and residual.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0
                and x.planes.data_ptr() % 16 == 0 and residual.device == x.device)
    if x.device.type != "cuda" or x.dtype not in (torch.bfloat16, torch.float16) or weight.dtype != x.dtype:
        return False
    hidden = int(x.shape[-1]) if x.dim() else 0
    if hidden == 0 or hidden % 8 or weight.numel() != hidden or not weight.is_contiguous():
        return False
    tensors = [x, weight] + ([residual] if residual is not None else [])
    if residual is not None and (residual.shape != x.shape or residual.dtype != x.dtype):
        return False
    return all(t.data_ptr() % 16 == 0 and (t.dim() < 2 or t.stride(-1) == 1) for t in tensors)


def rmsnorm(x: torch.Tensor | PartialSums, weight: torch.Tensor, eps: float,
            residual: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor | None]:
    """``(y, h)``: ``h = residual + x`` (rounded to the dtype; None without a residual) and
    ``y = RMSNorm(h or x) * weight``, in one kernel (``layers.py:14-31,185-195``). ``x`` may be
    a linear's :class:`PartialSums` (with a residual): the kernel adds them up first, bit for bit
    as the split-K reduction would have."""
    if isinstance(x, PartialSums):
        if residual is None:
            raise ValueError("partial sums need the residual add")
        shape = x.shape
        hidden = int(shape[-1])
        r2 = residual.reshape(-1, hidden).contiguous()
        rows = int(r2.shape[0])
        y = torch.empty(rows, hidden, dtype=x.dtype, device=x.device)
        h = torch.empty_like(y)
        bias = x.bias.contiguous() if x.bias is not None else None
        call(
            load_library().llmopt_rmsnorm_planes(
                x.planes.data_ptr(), int(x.planes.shape[0]), None if bias is None else bias.data_ptr(),
                r2.data_ptr(), hidden, h.data_ptr(), hidden, weight.data_ptr(), y.data_ptr(), hidden, rows, hidden,
                float(eps), DTYPE_CODES[x.dtype], _stream_handle(x.device),
            ),
            "llmopt_rmsnorm_planes",
        )
        return y.view(shape), h.view(shape)
    shape = x.shape
    hidden = int(shape[-1])
    x2 = x.reshape(-1, hidden)
    if x2.stride(-1) != 1 or x2.stride(0) % 8:
        x2 = x2.contiguous()
    r2 = residual.reshape(-1, hidden).contiguous() if residual is not None else None
    rows = int(x2.shape[0])
    y = torch.empty(rows, hidden, dtype=x.dtype, device=x.device)
    h = torch.empty_like(y) if residual is not None else None
    call(
        load_library().llmopt_rmsnorm(
            x2.data_ptr(), x2.stride(0), None if r2 is None else r2.data_ptr(), hidden,
            None if h is None else h.data_ptr(), hidden, weight.data_ptr(), y.data_ptr(), hidden, rows, hidden,
            float(eps), DTYPE_CODES[x.dtype], _stream_handle(x.device),
        ),
        "llmopt_rmsnorm",
    )
    return y.view(shape), (h.view(shape) if h is not None else None)


def rope(q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor, cos_table: torch.Tensor,
         sin_table: torch.Tensor, v: torch.Tensor | None = None) -> tuple[torch.Tensor, ...]:
    """Rotary embedding of ``q [tokens, heads, d]`` and ``k [tokens, kv_heads, d]`` (each with
    unit stride inside a token) at ``positions [tokens]``; returns new contiguous tensors,
    bit-identical to ``apply_rotary_pos_emb`` with the tables cast to the dtype. With ``v``
    (shaped like ``k``) a contiguous copy of it is returned third."""
    tokens, heads, d = (int(s) for s in q.shape)
    kv_heads = int(k.shape[1])

    def inner_ok(t: torch.Tensor) -> bool:
        return t.stride(2) == 1 and t.stride(1) == d

    if not inner_ok(q):
        q = q.contiguous()
    if not inner_ok(k):
        k = k.contiguous()
    if v is not None and not inner_ok(v):
        v = v.contiguous()
    pos = positions.to(device=q.device, dtype=torch.int64).contiguous()
    cos_t = cos_table.to(device=q.device, dtype=torch.float32).contiguous()
    sin_t = sin_table.to(device=q.device, dtype=torch.float32).contiguous()
    q_out = torch.empty(tokens, heads, d, dtype=q.dtype, device=q.device)
    k_out = torch.empty(tokens, kv_heads, d, dtype=k.dtype, device=k.device)
    v_out = torch.empty_like(k_out) if v is not None else None
    call(
        load_library().llmopt_rope(
            q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), None if v is None else v.data_ptr(),
            0 if v is None else v.stride(0), q_out.data_ptr(), k_out.data_ptr(),
            None if v_out is None else v_out.data_ptr(), pos.data_ptr(), cos_t.data_ptr(), sin_t.data_ptr(),
            int(cos_t.shape[0]), tokens, heads, kv_heads, d, DTYPE_CODES[q.dtype], _stream_handle(q.device),
        ),
        "llmopt_rope",
    )
    return (q_out, k_out) if v_out is None else (q_out, k_out, v_out)


def rope_kv_write_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, positions: torch.Tensor,
                         cos_table: torch.Tensor, sin_table: torch.Tensor, key_cache: torch.Tensor,
                         value_cache: torch.Tensor, block_ids: torch.Tensor,
                         token_offsets: torch.Tensor) -> torch.Tensor:
    """``rope`` for one token per sequence (``q [seqs, heads, d]``, ``k``/``v [seqs, kv_heads,
    d]``) with the rotated k and v stored straight into one layer's paged cache slots, as
    ``PagedKVCache.write_decode`` stores them (``paged_cache.py:246-277``); returns the rotated q.
    The cache must hold the activations' dtype."""
    seqs, heads, d = (int(s) for s in q.shape)
    kv_heads = int(k.shape[1])
    nb, bs, kvh, hd, _ = _layer_cache(key_cache, value_cache)
    if key_cache.dtype != q.dtype or (kvh, hd) != (kv_heads, d) or tuple(v.shape) != tuple(k.shape):
        raise ValueError("rope_kv_write_decode: cache dtype/shape does not match q/k/v")
    if int(k.shape[0]) != seqs or block_ids.dim() != 2:
        raise ValueError("rope_kv_write_decode: k/v need one row per query row, block_ids [seqs, blocks]")
    _check_rows("rope_kv_write_decode", seqs, positions=positions.reshape(-1),
                token_offsets=token_offsets.reshape(-1), block_ids=block_ids)

    def inner_ok(t: torch.Tensor) -> bool:
        return t.stride(2) == 1 and t.stride(1) == d

    q, k, v = (t if inner_ok(t) else t.contiguous() for t in (q, k, v))
    dev = q.device
    pos = positions.to(device=dev, dtype=torch.int64).contiguous()
    cos_t = cos_table.to(device=dev, dtype=torch.float32).contiguous()
    sin_t = sin_table.to(device=dev, dtype=torch.float32).contiguous()
    table = _int32(block_ids, dev)
    offsets = _int32(token_offsets, dev)
    q_out = torch.empty(seqs, heads, d, dtype=q.dtype, device=dev)
    call(
        load_library().llmopt_rope_kv_write_decode(
            q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0), q_out.data_ptr(),
            pos.data_ptr(), cos_t.data_ptr(), sin_t.data_ptr(), int(cos_t.shape[0]), seqs, heads, kv_heads, d,
            DTYPE_CODES[q.dtype], key_cache.data_ptr(), value_cache.data_ptr(), nb, bs, table.data_ptr(),
            int(table.shape[1]), offsets.data_ptr(), _stream_handle(dev),
        ),
        "llmopt_rope_kv_write_decode",
    )
    return q_out
