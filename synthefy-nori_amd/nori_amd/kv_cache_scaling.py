"""MI355X drop-in for ``synthefy_nori.model.kv_cache_scaling``: the int8 K/V cache codec and
the cache containers, with the reference's names, signatures, storage layout and exception
types (src/synthefy_nori/model/kv_cache_scaling.py) and every byte of arithmetic done by
libnori_hip.so.

* ``quantize_int8`` / ``dequantize_int8`` (reference :29-41) run the HIP codec; codes and
  scales are bit-identical to the reference torch expression evaluated on the GPU.
* The containers are built around the stored payload, ``KVRows``: a layer's rows as int8 codes
  + fp32 scales (or projected values) in the reference's ``[BG, N, 2, Hkv, D]`` layout, cut
  into row parts that are either views of one device allocation or pinned host blocks. The
  attention kernel reads that payload directly -- codes straight from HBM, dequantized in
  registers -- instead of the reference's full-layer dequantization on every ``cache["kv"]``
  read (:78-90). ``ScalableSeqKV`` (reference :44-178) keeps one joined payload and the
  reference's full-layer ``["kv"]`` read; ``BlockwiseSeqKV`` (reference :181-380) has no
  full-layer read and hands its rows out block by block, or as its one resident allocation.
* Device-resident int8 rows are coded slice by slice straight into their place in one
  allocation sized up front (two-level addressing in the kernel): no quantized slice exists
  outside the final storage and nothing is concatenated on the device.

There is no CPU path: quantizing or dequantizing a CPU tensor raises. Pure transport
(unquantized host blocks, offload copies) needs no kernel and works on any device.
"""

from __future__ import annotations

import torch

from . import _native as nat


# ----------------------------------------------------------------------------- helpers
def _vector_layout(t: torch.Tensor) -> tuple[int, int, int, int] | None:
    """Describe the head vectors (last axis) of ``t`` as (n_outer, n_inner, outer, inner) strides.

    Returns None when the leading axes do not collapse into two strided levels.
    """
    if t.dim() == 0 or t.stride(-1) != 1:
        return None
    sizes = list(t.shape[:-1])
    strides = list(t.stride()[:-1])
    # drop unit axes, they carry no addressing
    pairs = [(s, st) for s, st in zip(sizes, strides) if s != 1]
    if not pairs:
        return 1, 1, 0, t.shape[-1]
    # merge from the innermost leading axis outwards
    groups: list[list[int]] = [[pairs[-1][0], pairs[-1][1]]]
    for size, stride in reversed(pairs[:-1]):
        inner_size, inner_stride = groups[-1]
        if stride == inner_size * inner_stride:
            groups[-1][0] = inner_size * size
        else:
            groups.append([size, stride])
    if len(groups) == 1:
        n_inner, inner = groups[0]
        return 1, n_inner, 0, inner
    if len(groups) == 2:
        (n_inner, inner), (n_outer, outer) = groups
        return n_outer, n_inner, outer, inner
    return None


def _source_layout(t: torch.Tensor) -> tuple[torch.Tensor, tuple[int, int, int, int]]:
    layout = _vector_layout(t)
    if layout is None:
        t = t.contiguous()
        layout = _vector_layout(t)
    assert layout is not None
    return t, layout


def _split_strides(layout: tuple[int, int, int, int] | None, n_outer: int, n_inner: int) -> tuple[int, int] | None:
    """(outer, inner) strides addressing ``layout``'s vectors as an ``n_outer`` x ``n_inner`` grid.

    A single-level layout (vectors at k * inner) takes any split of its count; a two-level
    one only its own. None when the vectors cannot be addressed that way.
    """
    if layout is None:
        return None
    lo, li, so, si = layout
    if lo * li != n_outer * n_inner:
        return None
    if (lo, li) == (n_outer, n_inner):
        return so, si
    if lo == 1:
        return n_inner * si, si
    return None


def _quantize_into(src: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor) -> None:
    """Quantize ``src`` (float, last axis = head vector) into preallocated ``codes``/``scales`` views."""
    device = nat.require_device(src, codes, scales)
    if codes.dtype != torch.int8 or scales.dtype != torch.float32:
        raise ValueError("codes must be int8 and scales float32")
    if tuple(codes.shape) != tuple(src.shape) or tuple(scales.shape) != tuple(src.shape[:-1]) + (1,):
        raise ValueError(f"quantize_int8 output shapes {tuple(codes.shape)}/{tuple(scales.shape)} do not match {tuple(src.shape)}")
    if src.numel() == 0:
        return
    src, (so, si, sos, sis) = _source_layout(src)
    c_str = _split_strides(_vector_layout(codes), so, si)
    s_str = _split_strides(_vector_layout(scales), so, si)
    if c_str is None or s_str is None:
        # the destinations cannot be addressed with the source's vector grid: code into
        # contiguous buffers (always addressable) and copy
        tmp_c = torch.empty(src.shape, dtype=torch.int8, device=device)
        tmp_s = torch.empty(tuple(src.shape[:-1]) + (1,), dtype=torch.float32, device=device)
        _launch_quantize(src, (so, si, sos, sis), tmp_c, _split_strides(_vector_layout(tmp_c), so, si),
                         tmp_s, _split_strides(_vector_layout(tmp_s), so, si), device)
        codes.copy_(tmp_c)
        scales.copy_(tmp_s)
        return
    _launch_quantize(src, (so, si, sos, sis), codes, c_str, scales, s_str, device)


def _launch_quantize(src, src_layout, codes, c_str, scales, s_str, device) -> None:
    so, si, sos, sis = src_layout
    nat.check(
        nat.lib().nori_kv_quantize_int8(
            src.data_ptr(), nat.dtype_code(src.dtype), so, si, src.shape[-1], sos, sis,
            codes.data_ptr(), c_str[0], c_str[1],
            scales.data_ptr(), s_str[0], s_str[1],
            nat.SCALE_DIV_RECIP, nat.stream_of(device),
        ),
        "quantize_int8",
    )


def _dequantize_into(q: torch.Tensor, scale: torch.Tensor, out: torch.Tensor) -> None:
    device = nat.require_device(q, scale, out)
    if q.numel() == 0:
        return
    q, (qo, qi, qos, qis) = _source_layout(q)
    scale, s_layout = _source_layout(scale)
    s_str = _split_strides(s_layout, qo, qi)
    o_str = _split_strides(_vector_layout(out), qo, qi)
    if s_str is None:
        scale = scale.contiguous()
        s_str = _split_strides(_vector_layout(scale), qo, qi)
    target = out
    if o_str is None:
        target = torch.empty(q.shape, dtype=out.dtype, device=device)
        o_str = _split_strides(_vector_layout(target), qo, qi)
    nat.check(
        nat.lib().nori_kv_dequantize_int8(
            q.data_ptr(), scale.data_ptr(), qo, qi, q.shape[-1], qos, qis, s_str[0], s_str[1],
            target.data_ptr(), nat.dtype_code(out.dtype), o_str[0], o_str[1], nat.stream_of(device),
        ),
        "dequantize_int8",
    )
    if target is not out:
        out.copy_(target)


# ----------------------------------------------------------------------------- codec
def quantize_int8(t: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-vector (last-dim) absmax int8 quantization. Returns (int8, scale).

    scale has t's shape with the last dim = 1; dequant is q.float() * scale.
    Reference: kv_cache_scaling.py:29-37; bit-identical to it on the same GPU and dtype.
    """
    if t.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise NotImplementedError(f"quantize_int8 takes float32/float16/bfloat16, got {t.dtype}")
    nat.require_device(t)
    codes = torch.empty(t.shape, dtype=torch.int8, device=t.device)
    scale = torch.empty(tuple(t.shape[:-1]) + (1,), dtype=torch.float32, device=t.device)
    _quantize_into(t, codes, scale)
    return codes, scale


# ----------------------------------------------------------------------------- stored rows
# Largest int8 scale the attention kernel takes: it holds dequantized K/V as f16 values, and
# code * scale reaches 127 * scale, which must stay within f16's 65504. Scales of caches
# quantized from fp16 K/V (the GPU autocast path) are f16 values below it by construction;
# caches quantized from bf16 or fp32 K/V are checked the first time the kernel reads them.
# Scales below f16's normal range (2^-14) keep an absolute error under 127 * 2^-25 per element.
F16_SCALE_LIMIT = 65504.0 / 127.0


def _rows(payload: torch.Tensor) -> int:
    return int(payload.shape[1])


def _pinned_copy(t: torch.Tensor) -> torch.Tensor:
    """``t`` in host memory: a pinned copy of a device tensor (so staging it back is an
    asynchronous copy), or the host tensor itself when already there and contiguous."""
    t = t.detach()
    if t.device.type == "cpu":
        return t if t.is_contiguous() else t.contiguous()
    host = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    host.copy_(t)
    return host


class KVRows:
    """One layer's cached context K/V, ``[BG, N, 2, Hkv, D]``, stored as the payload the kernels read.

    * ``quantized``: int8 codes plus fp32 scales ``[BG, N, 2, Hkv, 1]`` (what the reference's
      ``quantize_int8`` returns, kv_cache_scaling.py:29-37); otherwise the projected values.
    * ``parts``: the payload cut along the row axis, in row order, as (payload, scales or None)
      pairs. Device-resident rows are views of one allocation, ``whole``, so the attention
      reads the layer in one launch and nothing is ever concatenated on the device; host rows
      are separate pinned blocks, staged onto the device one at a time (the host-offloaded
      and streamed caches of kv_cache_scaling.py:44-90, 181-358).
    * ``dtype``: the projected rows' dtype, which a dequantized read returns.
    """

    def __init__(self, parts, *, dtype: torch.dtype, device: torch.device, quantized: bool, on_host: bool, whole=None):
        parts = list(parts)
        if not parts:
            raise ValueError("a K/V cache needs at least one block of rows")
        self.parts = parts
        self.whole = whole
        self.dtype = dtype
        self.device = torch.device(device)
        self.quantized = bool(quantized)
        self.on_host = bool(on_host)
        self.n_rows = sum(_rows(p) for p, _ in parts)
        self.max_part_rows = max(_rows(p) for p, _ in parts)
        self._range_checked = not self.quantized or dtype == torch.float16

    # ------------------------------------------------------------------ building
    @classmethod
    def gather(cls, slices, *, quantize: bool, on_host: bool, device=None, dtype=None, n_rows: int | None = None,
               joined: bool = False) -> "KVRows":
        """Store projected row slices (``[BG, n, 2, Hkv, D]`` tensors, or ``FusedKVRows`` still to
        be projected), consumed one at a time in row order, so the full-precision layer never
        exists beyond one slice.

        * quantized on the device with ``n_rows`` known: one allocation for every row, each slice
          coded straight into its rows (int8 codes are per row, so slice-wise coding gives the
          whole-layer codes bit for bit);
        * otherwise each slice is stored as it comes -- in pinned host memory when ``on_host`` --
          and ``joined`` puts the parts back into one tensor at the end.
        """
        it = iter(slices)
        first = next(it, None)
        if first is None:
            raise ValueError("from_row_slices: no row slices, so there is nothing to cache")
        if dtype is None:
            dtype = first.dtype
        if device is None:
            device = first.device
        if quantize and not on_host and n_rows is not None:
            return cls._gather_in_place(first, it, device=torch.device(device), dtype=dtype, n_rows=n_rows)
        parts = []
        for kv_slice in _chain(first, it):
            if quantize:
                payload, scales = _quantize_slice(kv_slice)
            else:
                payload, scales = _projected(kv_slice), None
            if on_host:
                payload = _pinned_copy(payload)
                scales = None if scales is None else _pinned_copy(scales)
            elif payload.device != torch.device(device):
                payload = payload.to(device)
                scales = None if scales is None else scales.to(device)
            parts.append((payload, scales))
            del kv_slice, payload, scales
        whole = parts[0] if len(parts) == 1 else None
        if joined and whole is None:
            whole = (torch.cat([p for p, _ in parts], dim=1),
                     torch.cat([s for _, s in parts], dim=1) if quantize else None)
            parts = [whole]
        return cls(parts, dtype=dtype, device=device, quantized=quantize, on_host=on_host, whole=whole)

    @classmethod
    def _gather_in_place(cls, first, rest, *, device, dtype, n_rows: int) -> "KVRows":
        grid = tuple(first.shape)
        codes = torch.empty((grid[0], n_rows, *grid[2:]), dtype=torch.int8, device=device)
        scales = torch.empty((grid[0], n_rows, *grid[2:-1], 1), dtype=torch.float32, device=device)
        parts, row = [], 0
        for kv_slice in _chain(first, rest):
            width = int(kv_slice.shape[1])
            if row + width > n_rows:
                raise ValueError(f"row slices run past the n_rows={n_rows} the cache was sized for")
            view = (codes[:, row : row + width], scales[:, row : row + width])
            if isinstance(kv_slice, torch.Tensor):
                _quantize_into(kv_slice.to(device), *view)
            else:
                kv_slice.quantize_into(*view)
            parts.append(view)
            row += width
            del kv_slice
        if row != n_rows:
            raise ValueError(f"row slices hold {row} rows, but the cache was sized for n_rows={n_rows}")
        return cls(parts, dtype=dtype, device=device, quantized=True, on_host=False, whole=(codes, scales))

    # ------------------------------------------------------------------ reading
    def check_kernel_range(self) -> None:
        """Refuse int8 scales whose values the f16 attention kernel cannot hold (above
        F16_SCALE_LIMIT); runs once per cache, only for caches not quantized from fp16."""
        if self._range_checked:
            return
        top = max(float(s.amax()) for _, s in self.parts)
        if not top <= F16_SCALE_LIMIT:
            raise NotImplementedError(
                f"int8 cache scales reach {top:.4g}: its K/V values exceed the fp16 range (65504) the HIP "
                f"attention computes in (scales up to {F16_SCALE_LIMIT:.4g} are taken)"
            )
        self._range_checked = True

    def full(self) -> tuple[torch.Tensor, torch.Tensor | None]:
        """The whole layer's payload on the compute device (moved there when stored on the host)."""
        if self.whole is None:
            raise RuntimeError("these K/V rows are stored as separate blocks; read them block by block")
        payload, scales = self.whole
        if self.on_host:
            payload = payload.to(self.device, non_blocking=True)
            scales = None if scales is None else scales.to(self.device, non_blocking=True)
        return payload, scales

    def staged(self, block_rows: int | None):
        """(payload, scales) blocks of at most ``block_rows`` rows (the stored parts when None)
        on the compute device, in row order; only the block being yielded is staged."""
        if block_rows is not None and block_rows <= 0:
            raise ValueError("block_rows must be positive")
        for payload, scales in self.parts:
            n = _rows(payload)
            step = n if block_rows is None else min(block_rows, n)
            for r0 in range(0, n, step):
                r1 = min(r0 + step, n)
                # cut on the storage side, then move only the cut rows
                p = payload[:, r0:r1].to(self.device, non_blocking=True)
                s = None if scales is None else scales[:, r0:r1].to(self.device, non_blocking=True)
                yield p, s
                del p, s

    def bytes_where(self, on_host: bool) -> int:
        if self.on_host != on_host:
            return 0
        total = 0
        for payload, scales in self.parts:
            total += payload.numel() * payload.element_size()
            if scales is not None:
                total += scales.numel() * scales.element_size()
        return total


def _chain(first, rest):
    yield first
    yield from rest


def _quantize_slice(kv_slice) -> tuple[torch.Tensor, torch.Tensor]:
    """Codes and scales of a projected row slice, or of a ``FusedKVRows`` slice that one kernel
    projects and quantizes (nori_amd.kv_project)."""
    if isinstance(kv_slice, torch.Tensor):
        return quantize_int8(kv_slice)
    return kv_slice.quantize()


def _projected(kv_slice) -> torch.Tensor:
    if isinstance(kv_slice, torch.Tensor):
        return kv_slice.detach()
    raise TypeError("a fused projection slice is only ever stored as an int8 cache (quantize=True)")


def dequantize_int8(q: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """(q.float() * scale).to(dtype) -- reference kv_cache_scaling.py:40-41."""
    if dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise NotImplementedError(f"dequantize_int8 produces float32/float16/bfloat16, got {dtype}")
    if q.dtype != torch.int8:
        raise ValueError(f"dequantize_int8 expects int8 codes, got {q.dtype}")
    nat.require_device(q, scale)
    out = torch.empty(q.shape, dtype=dtype, device=q.device)
    _dequantize_into(q, scale.to(torch.float32), out)
    return out


# ----------------------------------------------------------------------------- caches
class ScalableSeqKV:
    """Whole-layer seq-attn cache, dict-like ``{"kv", "batch", "groups"}`` (reference
    kv_cache_scaling.py:44-178), int8 and/or host-resident.

    The stored rows are a ``KVRows`` held as one payload. The attention operators of this
    package read it through ``device_payload()`` and dequantize inside the kernel;
    ``cache["kv"]`` is the full-precision layer the reference's readers expect, dequantized by
    the HIP codec (and moved, when offloaded) on each read.
    """

    def __init__(self, kv: torch.Tensor, batch: int, groups: int, *, quantize: bool = False, offload: bool = False,
                 device: torch.device | None = None):
        target = torch.device(device) if device is not None else kv.device
        rows = KVRows.gather([kv], quantize=quantize, on_host=offload, device=target, dtype=kv.dtype,
                             n_rows=int(kv.shape[1]), joined=True)
        self._bind(rows, batch, groups)

    def _bind(self, rows: KVRows, batch: int, groups: int) -> None:
        self.rows = rows
        self.batch = int(batch)
        self.groups = int(groups)

    @classmethod
    def from_payload(cls, payload: torch.Tensor, scales: torch.Tensor | None, batch: int, groups: int, *,
                     dtype: torch.dtype | None = None, offload: bool = False) -> "ScalableSeqKV":
        """Wrap stored rows as they are: int8 codes with their fp32 scales (``dtype`` names what
        they dequantize to), or full-precision values (``scales`` None)."""
        quantized = scales is not None
        if quantized and (payload.dtype != torch.int8 or scales.dtype != torch.float32):
            raise ValueError("an int8 payload needs int8 codes and float32 scales")
        obj = cls.__new__(cls)
        rows = KVRows([(payload, scales)], dtype=dtype or (torch.float32 if quantized else payload.dtype),
                      device=payload.device, quantized=quantized, on_host=offload, whole=(payload, scales))
        obj._bind(rows, batch, groups)
        return obj

    @classmethod
    def from_row_slices(cls, slices, batch: int, groups: int, *, quantize: bool = False, offload: bool = False,
                        device: torch.device | None = None, dtype: torch.dtype | None = None) -> "ScalableSeqKV":
        """The cache of row-axis slices taken in order (reference :92-170): each slice is coded
        or moved as it arrives, so only one full-precision slice exists at a time; the stored
        parts are joined into one payload at the end (int8 codes are per row, so they join to
        the whole-layer codes bit for bit).

        Raises:
            ValueError: if ``slices`` is empty.
        """
        rows = KVRows.gather(slices, quantize=quantize, on_host=offload, device=device, dtype=dtype, joined=True)
        obj = cls.__new__(cls)
        obj._bind(rows, batch, groups)
        return obj

    # -- the reference's attributes
    @property
    def device(self) -> torch.device:
        return self.rows.device

    @property
    def dtype(self) -> torch.dtype:
        return self.rows.dtype

    @property
    def quantized(self) -> bool:
        return self.rows.quantized

    @property
    def offloaded(self) -> bool:
        return self.rows.on_host

    @property
    def n_rows(self) -> int:
        return self.rows.n_rows

    def __getitem__(self, key: str):
        if key == "batch":
            return self.batch
        if key == "groups":
            return self.groups
        if key == "kv":
            payload, scales = self.rows.full()
            return dequantize_int8(payload, scales, self.dtype) if self.quantized else payload
        raise KeyError(key)

    def device_payload(self) -> tuple[torch.Tensor, torch.Tensor | None]:
        """(payload, scales) on the compute device: int8 codes + fp32 scales, or (values, None)."""
        self.rows.check_kernel_range()
        return self.rows.full()

    def resident_gpu_bytes(self) -> int:
        """Bytes held on the compute device between reads (0 when offloaded)."""
        return self.rows.bytes_where(on_host=False)


class BlockwiseSeqKV:
    """Bounded-device seq-attn cache (reference kv_cache_scaling.py:181-380): the layer is never
    materialized on the device, ``cache["kv"]`` raises, and readers take blocks of rows.

    The stored rows are a ``KVRows``: pinned host blocks staged one at a time (host-streamed), or
    one device allocation of int8 codes filled slice by slice (resident). The attention reads a
    resident cache in one launch (``resident_payload``) and streams a host one block by block
    with exact LSE merging (``host_blocks``); ``iter_kv_blocks`` gives the reference's
    dequantized blocks.
    """

    def __init__(self, blocks, batch: int, groups: int, *, device: torch.device, dtype: torch.dtype, quantized: bool,
                 offloaded: bool = True):
        self._bind(KVRows(blocks, dtype=dtype, device=device, quantized=quantized, on_host=offloaded), batch, groups)

    def _bind(self, rows: KVRows, batch: int, groups: int) -> None:
        self.rows = rows
        self.batch = int(batch)
        self.groups = int(groups)
        # rows of the largest block staged by the last scan (a report of the bound held)
        self.max_staged_rows = 0

    @classmethod
    def from_row_slices(cls, slices, batch: int, groups: int, *, quantize: bool, device: torch.device,
                        dtype: torch.dtype | None = None, offload: bool = True,
                        n_rows: int | None = None) -> "BlockwiseSeqKV":
        """The cache of row-axis slices taken in order (reference :232-330), with no
        concatenation: host-streamed caches keep one pinned block per slice; resident caches are
        int8, sized by ``n_rows`` up front and coded slice by slice into their rows."""
        if not offload:
            if not quantize:
                raise ValueError("a device-resident blockwise cache is stored as int8 (quantize=True)")
            if n_rows is None or n_rows <= 0:
                raise ValueError("a device-resident blockwise cache must be sized by a positive n_rows")
        rows = KVRows.gather(slices, quantize=quantize, on_host=offload, device=device, dtype=dtype,
                             n_rows=None if offload else int(n_rows))
        obj = cls.__new__(cls)
        obj._bind(rows, batch, groups)
        return obj

    # -- the reference's attributes
    @property
    def device(self) -> torch.device:
        return self.rows.device

    @property
    def dtype(self) -> torch.dtype:
        return self.rows.dtype

    @property
    def quantized(self) -> bool:
        return self.rows.quantized

    @property
    def offloaded(self) -> bool:
        return self.rows.on_host

    @property
    def n_rows(self) -> int:
        return self.rows.n_rows

    @property
    def max_block_rows(self) -> int:
        return self.rows.max_part_rows

    def __getitem__(self, key: str):
        if key == "batch":
            return self.batch
        if key == "groups":
            return self.groups
        if key == "kv":
            raise RuntimeError(
                "BlockwiseSeqKV cannot materialize a full layer on the compute device: its rows are read "
                "block by block (iter_kv_blocks, or the HIP attention's blockwise scan)"
            )
        raise KeyError(key)

    def _scan(self, block_rows: int | None):
        self.max_staged_rows = 0
        for payload, scales in self.rows.staged(block_rows):
            self.max_staged_rows = max(self.max_staged_rows, _rows(payload))
            yield payload, scales

    def iter_kv_blocks(self, block_rows: int | None = None):
        """Full-precision K/V blocks on the compute device, in row order."""
        for payload, scales in self._scan(block_rows):
            yield dequantize_int8(payload, scales, self.dtype) if self.quantized else payload

    def iter_payload_blocks(self, block_rows: int | None = None):
        """(payload, scales or None) blocks on the compute device, not dequantized."""
        self.rows.check_kernel_range()
        yield from self._scan(block_rows)

    def host_blocks(self) -> list[tuple[torch.Tensor, torch.Tensor | None]]:
        """The stored (payload, scales or None) host blocks in row order: what the overlapped
        streamed scan stages itself."""
        if not self.offloaded:
            raise RuntimeError("host_blocks() is for host-offloaded caches; use resident_payload()")
        self.rows.check_kernel_range()
        return list(self.rows.parts)

    def device_blocks(self) -> list[tuple[torch.Tensor, torch.Tensor | None]]:
        """The stored (payload, scales or None) blocks of a device-resident cache, in row order."""
        if self.offloaded:
            raise RuntimeError("device_blocks() is for device-resident caches; use host_blocks()")
        self.rows.check_kernel_range()
        return list(self.rows.parts)

    def resident_payload(self) -> tuple[torch.Tensor, torch.Tensor] | None:
        """The whole device-resident payload and scales (one allocation), else None."""
        if self.offloaded or self.rows.whole is None:
            return None
        self.rows.check_kernel_range()
        return self.rows.whole

    def resident_gpu_bytes(self) -> int:
        """Bytes held on the compute device between scans."""
        return self.rows.bytes_where(on_host=False)

    def host_bytes(self) -> int:
        """Bytes held in host memory."""
        return self.rows.bytes_where(on_host=True)


def scale_caches(caches: list[dict], *, quantize: bool = False, offload: bool = False,
                 device: torch.device | None = None) -> list[dict]:
    """Store every layer's ``seq_kv`` dict as a ScalableSeqKV, int8 and/or host-resident, in
    place (reference :383-404). Nothing to do when neither is asked; caches already converted,
    and caches without a ``kv`` entry, are left as they are."""
    if quantize or offload:
        for layer_cache in caches:
            entry = layer_cache.get("seq_kv")
            if isinstance(entry, dict) and "kv" in entry:
                layer_cache["seq_kv"] = ScalableSeqKV(entry["kv"], entry["batch"], entry["groups"], quantize=quantize,
                                                      offload=offload, device=device)
    return caches
