"""MI355X drop-in for ``synthefy_nori.model.kv_cache_scaling``.

Same names, signatures, storage layouts and error behaviour as the reference module
(src/synthefy_nori/model/kv_cache_scaling.py), with every byte of arithmetic done by
libnori_hip.so:

* ``quantize_int8`` / ``dequantize_int8`` (reference :29-41) run the HIP codec, whose
  codes and scales are bit-identical to the reference torch expression evaluated on the
  GPU.
* ``ScalableSeqKV`` (reference :44-178) and ``BlockwiseSeqKV`` (reference :181-380) keep
  the reference's payload layout ``[BG, N, 2, Hkv, D]`` int8 + ``[BG, N, 2, Hkv, 1]`` fp32.
  They additionally expose the int8 payload itself (``device_payload``,
  ``iter_payload_blocks``, ``resident_payload``) so the attention kernel reads codes
  straight from HBM instead of re-dequantizing the whole layer for every query chunk
  (the reference's ``cache["kv"]`` read, :78-90).
* Resident int8 blockwise storage is filled in place: each slice is quantized straight
  into its rows of the preallocated payload (two-level addressing in the kernel), so not
  even one quantized slice is materialized outside the final storage.

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


def _quantize_slice(kv_slice) -> tuple[torch.Tensor, torch.Tensor]:
    """Codes and scales of a projected row slice, or of a ``FusedKVRows`` slice that is projected
    and quantized by one kernel (nori_amd.kv_project)."""
    if isinstance(kv_slice, torch.Tensor):
        return quantize_int8(kv_slice)
    return kv_slice.quantize()


def _projected(kv_slice) -> torch.Tensor:
    if isinstance(kv_slice, torch.Tensor):
        return kv_slice
    raise TypeError("a fused projection slice only builds an int8 cache (quantize=True)")


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
    """Dict-like drop-in for the ``{"kv","batch","groups"}`` seq-attn cache.

    Stores ``kv`` int8-quantized and/or on host RAM; ``self["kv"]`` returns the
    full-precision tensor on ``device`` (dequantized + moved). Reference
    kv_cache_scaling.py:44-178. The attention operators of this package do not read
    ``["kv"]``: they take ``device_payload()`` and dequantize inside the kernel.
    """

    def __init__(
        self,
        kv: torch.Tensor,
        batch: int,
        groups: int,
        *,
        quantize: bool = False,
        offload: bool = False,
        device: torch.device | None = None,
    ):
        self.batch = int(batch)
        self.groups = int(groups)
        self.device = torch.device(device) if device is not None else kv.device
        self.dtype = kv.dtype
        self.quantized = quantize
        self.offloaded = offload
        store_dev = torch.device("cpu") if offload else self.device
        if quantize:
            q, scale = quantize_int8(kv)
            self._q = q.to(store_dev, non_blocking=False)
            self._scale = scale.to(store_dev, non_blocking=False)
            self._kv = None
        else:
            self._q = self._scale = None
            self._kv = kv.to(store_dev, non_blocking=False)

    def __getitem__(self, key: str):
        if key == "batch":
            return self.batch
        if key == "groups":
            return self.groups
        if key == "kv":
            if self.quantized:
                q, scale = self.device_payload()
                return dequantize_int8(q, scale, self.dtype)
            kv = self._kv
            return kv.to(self.device, non_blocking=True) if self.offloaded else kv
        raise KeyError(key)

    def device_payload(self) -> tuple[torch.Tensor, torch.Tensor | None]:
        """(payload, scale) on the compute device: int8 codes + fp32 scales, or (kv, None)."""
        if self.quantized:
            q = self._q.to(self.device, non_blocking=True) if self.offloaded else self._q
            s = self._scale.to(self.device, non_blocking=True) if self.offloaded else self._scale
            return q, s
        kv = self._kv.to(self.device, non_blocking=True) if self.offloaded else self._kv
        return kv, None

    @property
    def n_rows(self) -> int:
        return int((self._q if self.quantized else self._kv).shape[1])

    @classmethod
    def from_row_slices(
        cls,
        slices,
        batch: int,
        groups: int,
        *,
        quantize: bool = False,
        offload: bool = False,
        device: torch.device | None = None,
        dtype: torch.dtype | None = None,
    ) -> "ScalableSeqKV":
        """Build from row-axis slices, quantizing/moving each one as it arrives (reference :92-170).

        Quantization is per (row, head) vector, so per-slice codes concatenate to the
        whole-tensor codes bit for bit.

        Raises:
            ValueError: if ``slices`` is empty.
        """
        store = torch.device("cpu") if offload else None
        q_parts: list[torch.Tensor] = []
        scale_parts: list[torch.Tensor] = []
        kv_parts: list[torch.Tensor] = []
        for kv_slice in slices:
            if dtype is None:
                dtype = kv_slice.dtype
            if device is None:
                device = kv_slice.device
            if quantize:
                q, scale = _quantize_slice(kv_slice)
                q_parts.append(q if store is None else q.to(store))
                scale_parts.append(scale if store is None else scale.to(store))
            else:
                kv_parts.append(_projected(kv_slice) if store is None else _projected(kv_slice).to(store))
        if not (q_parts or kv_parts):
            raise ValueError("from_row_slices got no slices; nothing to cache")

        obj = cls.__new__(cls)
        obj.batch = int(batch)
        obj.groups = int(groups)
        obj.device = device if device is not None else torch.device("cpu")
        obj.dtype = dtype
        obj.quantized = bool(quantize)
        obj.offloaded = bool(offload)
        if quantize:
            obj._q = torch.cat(q_parts, dim=1)
            obj._scale = torch.cat(scale_parts, dim=1)
            obj._kv = None
        else:
            obj._q = obj._scale = None
            obj._kv = torch.cat(kv_parts, dim=1)
        return obj

    def resident_gpu_bytes(self) -> int:
        """Bytes this cache holds resident on the GPU (0 if offloaded)."""
        if self.offloaded:
            return 0
        if self.quantized:
            return self._q.numel() + self._scale.numel() * 4
        return self._kv.numel() * self._kv.element_size()


class BlockwiseSeqKV:
    """Blockwise K/V storage for bounded-device attention (reference :181-380).

    Host-streamed blocks live in pinned host memory; the resident int8 form is one
    preallocated device payload exposed as disjoint row views. ``cache["kv"]`` raises;
    consumers iterate blocks (``iter_kv_blocks`` for dequantized blocks, or
    ``iter_payload_blocks`` / ``resident_payload`` for the raw int8 payload that the
    attention kernel dequantizes in registers).
    """

    def __init__(
        self,
        blocks: list[tuple[torch.Tensor, torch.Tensor | None]],
        batch: int,
        groups: int,
        *,
        device: torch.device,
        dtype: torch.dtype,
        quantized: bool,
        offloaded: bool = True,
        _storage: tuple[torch.Tensor, torch.Tensor] | None = None,
    ):
        if not blocks:
            raise ValueError("BlockwiseSeqKV requires at least one K/V block")
        self.batch = int(batch)
        self.groups = int(groups)
        self.device = torch.device(device)
        self.dtype = dtype
        self.quantized = bool(quantized)
        self.offloaded = bool(offloaded)
        self._blocks = blocks
        self._storage = _storage
        self.n_rows = sum(int(payload.shape[1]) for payload, _ in blocks)
        self.max_block_rows = max(int(payload.shape[1]) for payload, _ in blocks)
        # Diagnostic used by reports/tests. It is reset at the start of each scan.
        self.max_staged_rows = 0

    def __getitem__(self, key: str):
        if key == "batch":
            return self.batch
        if key == "groups":
            return self.groups
        if key == "kv":
            raise RuntimeError(
                "BlockwiseSeqKV cannot materialize a full layer on the compute "
                "device; consume iter_kv_blocks() with online-softmax attention"
            )
        raise KeyError(key)

    @classmethod
    def from_row_slices(
        cls,
        slices,
        batch: int,
        groups: int,
        *,
        quantize: bool,
        device: torch.device,
        dtype: torch.dtype | None = None,
        offload: bool = True,
        n_rows: int | None = None,
    ) -> "BlockwiseSeqKV":
        """Consume projected row slices without a concatenation peak (reference :232-330).

        Resident int8 caches preallocate the final payload and scales once and quantize
        each slice directly into its rows. Host-offloaded caches keep one pinned host
        block per slice.
        """
        if not offload:
            if not quantize:
                raise ValueError("resident blockwise K/V requires quantize=True")
            if n_rows is None or n_rows <= 0:
                raise ValueError("resident blockwise K/V requires a positive n_rows")
            iterator = iter(slices)
            try:
                first_slice = next(iterator)
            except StopIteration as exc:
                raise ValueError("from_row_slices got no slices; nothing to cache") from exc
            if dtype is None:
                dtype = first_slice.dtype
            target_device = torch.device(device)
            payload_shape = (first_slice.shape[0], n_rows, *first_slice.shape[2:])
            scale_shape = (first_slice.shape[0], n_rows, *first_slice.shape[2:-1], 1)
            payload_storage = torch.empty(payload_shape, dtype=torch.int8, device=target_device)
            scale_storage = torch.empty(scale_shape, dtype=torch.float32, device=target_device)
            blocks: list[tuple[torch.Tensor, torch.Tensor | None]] = []
            offset = 0

            def store(kv_slice: torch.Tensor) -> None:
                nonlocal offset
                width = int(kv_slice.shape[1])
                end = offset + width
                if end > n_rows:
                    raise ValueError(f"row slices exceed declared n_rows={n_rows}")
                payload_view = payload_storage[:, offset:end]
                scale_view = scale_storage[:, offset:end]
                if isinstance(kv_slice, torch.Tensor):
                    _quantize_into(kv_slice.to(target_device), payload_view, scale_view)
                else:
                    kv_slice.quantize_into(payload_view, scale_view)
                blocks.append((payload_view, scale_view))
                offset = end

            store(first_slice)
            del first_slice
            for kv_slice in iterator:
                store(kv_slice)
                del kv_slice
            if offset != n_rows:
                raise ValueError(f"row slices covered {offset} rows, expected n_rows={n_rows}")
            return cls(
                blocks,
                batch,
                groups,
                device=target_device,
                dtype=dtype,
                quantized=True,
                offloaded=False,
                _storage=(payload_storage, scale_storage),
            )

        blocks = []
        for kv_slice in slices:
            if dtype is None:
                dtype = kv_slice.dtype
            if quantize:
                payload, scale = _quantize_slice(kv_slice)
                blocks.append((_to_host(payload), _to_host(scale)))
                del payload, scale
            else:
                blocks.append((_to_host(_projected(kv_slice).detach()), None))
            del kv_slice
        if dtype is None:
            raise ValueError("from_row_slices got no slices; nothing to cache")
        return cls(blocks, batch, groups, device=device, dtype=dtype, quantized=quantize, offloaded=True)

    def _staged_blocks(self, block_rows: int | None):
        if block_rows is not None and block_rows <= 0:
            raise ValueError("block_rows must be positive")
        self.max_staged_rows = 0
        for payload, stored_scale in self._blocks:
            stored_rows = int(payload.shape[1])
            step = stored_rows if block_rows is None else min(block_rows, stored_rows)
            for start in range(0, stored_rows, step):
                end = min(start + step, stored_rows)
                # Slice while still on the host; only this block is staged.
                staged_payload = payload[:, start:end].to(self.device, non_blocking=True)
                staged_scale = None
                if self.quantized:
                    assert stored_scale is not None
                    staged_scale = stored_scale[:, start:end].to(self.device, non_blocking=True)
                self.max_staged_rows = max(self.max_staged_rows, end - start)
                yield staged_payload, staged_scale
                del staged_payload, staged_scale

    def iter_kv_blocks(self, block_rows: int | None = None):
        """Yield full-precision K/V blocks on the compute device, in row order."""
        for payload, scale in self._staged_blocks(block_rows):
            yield dequantize_int8(payload, scale, self.dtype) if self.quantized else payload

    def iter_payload_blocks(self, block_rows: int | None = None):
        """Yield (payload, scale-or-None) blocks on the compute device without dequantizing."""
        yield from self._staged_blocks(block_rows)

    def host_blocks(self) -> list[tuple[torch.Tensor, torch.Tensor | None]]:
        """The stored (payload, scale-or-None) blocks of a host-offloaded cache, in row order: the
        source of the overlapped streamed scan, which stages them itself."""
        if not self.offloaded:
            raise RuntimeError("host_blocks() is for host-offloaded caches; use resident_payload()")
        return list(self._blocks)

    def resident_payload(self) -> tuple[torch.Tensor, torch.Tensor] | None:
        """The whole resident int8 payload and scales, when the cache is device resident."""
        if self.offloaded or self._storage is None:
            return None
        return self._storage

    def resident_gpu_bytes(self) -> int:
        """Bytes retained on the compute device between iterator steps."""
        if self.offloaded:
            return 0
        total = 0
        for payload, scale in self._blocks:
            total += payload.numel() * payload.element_size()
            if scale is not None:
                total += scale.numel() * scale.element_size()
        return total

    def host_bytes(self) -> int:
        """Bytes retained by the host block list."""
        if not self.offloaded:
            return 0
        total = 0
        for payload, scale in self._blocks:
            total += payload.numel() * payload.element_size()
            if scale is not None:
                total += scale.numel() * scale.element_size()
        return total


def _to_host(t: torch.Tensor) -> torch.Tensor:
    """Copy to host memory; pinned when the source is on a GPU so later H2D staging is async."""
    if t.device.type == "cpu":
        return t.detach().clone() if not t.is_contiguous() else t.detach()
    host = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    host.copy_(t.detach())
    return host


def scale_caches(
    caches: list[dict], *, quantize: bool = False, offload: bool = False, device: torch.device | None = None
) -> list[dict]:
    """Wrap each layer cache's ``seq_kv`` in a ScalableSeqKV (in place), reference :383-404."""
    if not (quantize or offload):
        return caches
    for layer_cache in caches:
        skv = layer_cache.get("seq_kv")
        if skv is None or isinstance(skv, (ScalableSeqKV, BlockwiseSeqKV)):
            continue
        if "kv" not in skv:
            continue
        layer_cache["seq_kv"] = ScalableSeqKV(
            skv["kv"],
            skv["batch"],
            skv["groups"],
            quantize=quantize,
            offload=offload,
            device=device,
        )
    return caches
