"""Host-side interface of the GPU MoE layer.

Mirrors the reference's layer-call seam (inspirewind/Urbilateria 0.2.4):
``MoeLayer.forward(input) -> (output, routes)`` is the return shape of
``RuntimeMoeLayer::forward`` (src/models/glm/runtime/moe.rs:138-176) and of
``execute_streamed_moe`` / ``execute_batched_moe`` (src/models/qwen3_6/runtime.rs:1067-1243):
token-major ``[tokens, hidden]`` f32 in and out, routes per token in ranking order, and an
exception (``UrbError``, the Result's Err) carrying the reference's error kind.  All compute
runs in ``liburb_moe.so`` through the C ABI; this module only owns device buffers.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional, Tuple

import numpy as np

from . import configs as C
from . import native as N
from . import synth

try:  # torch provides device memory and streams (plumbing only)
    import torch
except Exception:  # pragma: no cover
    torch = None

Pair = Tuple[object, Optional[object]]


def _ptr(t) -> Optional[int]:
    if t is None:
        return None
    if isinstance(t, np.ndarray):
        assert t.flags["C_CONTIGUOUS"]
        return t.ctypes.data
    assert t.is_contiguous()
    return t.data_ptr()


def _stream_handle(stream=None) -> Optional[int]:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream or None


@dataclass
class DeviceLayer:
    """One layer's weights resident in HBM in the reference's on-disk layouts (torch tensors
    viewing a single arena allocation)."""
    spec: C.LayerSpec
    router_weight: "torch.Tensor"                 # [E, H] int16 (BF16 bits)
    experts: List[List[Pair]]                     # [E][gate, up, down] (data, scales)
    shared: Optional[List[Pair]]
    correction_bias: Optional["torch.Tensor"]     # [E] f32
    arena: Optional["torch.Tensor"] = None
    shared_expert_gate: Optional["torch.Tensor"] = None  # [H] int16 BF16 (QWEN36 shared expert)
    hash_experts: Optional["torch.Tensor"] = None  # [vocab, k] int64 tid2eid (sqrt-softplus)

    @staticmethod
    def from_host(host: C.HostLayer, device="cuda") -> "DeviceLayer":
        def up(a):
            return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(device)
        ex = [[(up(d), up(s)) for d, s in trip] for trip in host.experts]
        sh = None if host.shared is None else [(up(d), up(s)) for d, s in host.shared]
        rw = torch.from_numpy(host.router_weight.view(np.int16)).to(device)
        bias = up(host.correction_bias)
        gate = None
        if host.shared_expert_gate is not None:
            gate = torch.from_numpy(host.shared_expert_gate.view(np.int16)).to(device)
        return DeviceLayer(host.spec, rw, ex, sh, bias, shared_expert_gate=gate,
                           hash_experts=up(host.hash_experts))

    @staticmethod
    def synthesize(spec: C.LayerSpec, base_seed: int = synth.BASE_SEED,
                   correction_bias: Optional[np.ndarray] = None, device="cuda",
                   stream=None) -> "DeviceLayer":
        """Generates the seeded layer directly in HBM with the device generator (the same
        streams as ``configs.make_host_layer``)."""
        lib = N.synth_lib()
        H, I, E, Is = spec.hidden, spec.intermediate, spec.n_experts, spec.shared_intermediate
        mats = []  # (name, fmt, rows, cols)
        for e in range(E):
            mats += [(f"expert.{e}.gate", spec.expert_format, I, H),
                     (f"expert.{e}.up", spec.expert_format, I, H),
                     (f"expert.{e}.down", spec.expert_format, H, I)]
        if Is:
            mats += [("shared.gate", spec.shared_format, Is, H),
                     ("shared.up", spec.shared_format, Is, H),
                     ("shared.down", spec.shared_format, H, Is)]
        al = lambda n: (n + 255) // 256 * 256
        qwen_gate = bool(Is) and spec.composition == C.COMPOSE_QWEN36
        total = al(E * H * 2) + (al(H * 2) if qwen_gate else 0)
        for _, fmt, r, c in mats:
            db, sb = C.matrix_bytes(fmt, r, c)
            total += al(db) + al(sb)
        arena = torch.empty(total, dtype=torch.uint8, device=device)
        s = _stream_handle(stream)
        off = 0

        def take(n):
            nonlocal off
            t = arena[off:off + n]
            off += al(n)
            return t

        rw = take(E * H * 2)
        N.check(lib.urb_synth_bf16(synth.stream_seed("router", base_seed), E * H, 0.0, 0.02,
                                   rw.data_ptr(), s), "synth router")
        out = []
        for name, fmt, r, c in mats:
            db, sb = C.matrix_bytes(fmt, r, c)
            d = take(db)
            sc = take(sb) if sb else None
            seed = synth.stream_seed(name, base_seed)
            if fmt == C.FMT_BF16:
                N.check(lib.urb_synth_bf16(seed, r * c, 0.0, 0.02, d.data_ptr(), s), name)
            elif fmt == C.FMT_MXFP4:
                N.check(lib.urb_synth_fp4(seed, db, d.data_ptr(), s), name)
            else:
                N.check(lib.urb_synth_fp8(seed, db, d.data_ptr(), s), name)
            if sc is not None:
                N.check(lib.urb_synth_e8m0(synth.stream_seed(name + ".scales", base_seed), sb,
                                           sc.data_ptr(), s), name)
            out.append((d, sc))
        ex = [out[3 * e:3 * e + 3] for e in range(E)]
        sh = out[3 * E:3 * E + 3] if Is else None
        gate = None
        if qwen_gate:
            gate = take(H * 2)
            N.check(lib.urb_synth_bf16(synth.stream_seed("shared.expert_gate", base_seed), H, 0.0,
                                       0.02, gate.data_ptr(), s), "synth shared expert gate")
            gate = gate.view(torch.int16)
        bias = None
        if correction_bias is not None:
            bias = torch.from_numpy(np.ascontiguousarray(correction_bias, np.float32)).to(device)
        return DeviceLayer(spec, rw.view(torch.int16).view(E, H), ex, sh, bias, arena, gate)

    @staticmethod
    def from_consolidated(spec: C.LayerSpec, router_weight, gate_up, gate_up_scales, down,
                          down_scales, shared: Optional[List[Pair]] = None,
                          correction_bias=None, shared_expert_gate=None,
                          hash_experts=None) -> "DeviceLayer":
        """A layer over consolidated expert tensors, used in place: gate_up [E, 2I, H] (each
        expert's gate rows, then its up rows) and down [E, H, I] in the on-disk layouts, scales
        [E, 2I, H/32] and [E, H, I/32] for the MX formats (None for BF16) -- the Qwen3.6 packed
        BF16 and Hy4 consolidated E4M3 + U8 checkpoints.  The per-expert views are the ones
        ``urb_expert_views`` computes for C callers."""
        E, I = spec.n_experts, spec.intermediate
        if gate_up.shape[0] != E or gate_up.shape[1] != 2 * I or down.shape[0] != E:
            raise ValueError("consolidated tensors do not match the layer geometry")
        ex = []
        for e in range(E):
            gs = None if gate_up_scales is None else gate_up_scales[e, :I]
            us = None if gate_up_scales is None else gate_up_scales[e, I:]
            ds = None if down_scales is None else down_scales[e]
            ex.append([(gate_up[e, :I], gs), (gate_up[e, I:], us), (down[e], ds)])
        return DeviceLayer(spec, router_weight, ex, shared, correction_bias,
                           shared_expert_gate=shared_expert_gate, hash_experts=hash_experts)

    def to_host(self, experts: Optional[List[int]] = None) -> C.HostLayer:
        """Copies (a subset of) the layer back to host memory for the CPU oracle."""
        def down(t):
            return None if t is None else t.cpu().numpy()
        keep = range(self.spec.n_experts) if experts is None else set(experts)
        ex = []
        for e, trip in enumerate(self.experts):
            ex.append([(down(d), down(s)) for d, s in trip] if e in keep else None)
        sh = None if self.shared is None else [(down(d), down(s)) for d, s in self.shared]
        rw = self.router_weight.contiguous().cpu().numpy().view(np.uint16).reshape(
            self.spec.n_experts, self.spec.hidden)
        bias = None if self.correction_bias is None else self.correction_bias.cpu().numpy()
        gate = None
        if self.shared_expert_gate is not None:
            gate = self.shared_expert_gate.cpu().numpy().view(np.uint16).reshape(-1)
        return C.HostLayer(self.spec, rw, ex, sh, bias, gate, down(self.hash_experts))


class MoeLayer:
    """A GPU MoE layer (``urb_moe_ctx``)."""

    def __init__(self, layer, max_tokens: int, source: Optional[int] = None):
        spec: C.LayerSpec = layer.spec
        self.spec = spec
        self.max_tokens = max_tokens
        lib = N.moe_lib()
        E = spec.n_experts
        host = isinstance(layer, C.HostLayer)
        if source is None:
            source = N.SOURCE_HOST if host else N.SOURCE_DEVICE_COPY
        # borrowed (panel-layout) buffers must outlive the context; copies do not
        self._layer = layer if source == N.SOURCE_DEVICE_BORROW else None
        mats = (N.Matrix * (3 * E))()
        for e in range(E):
            for m in range(3):
                d, s = layer.experts[e][m]
                mats[3 * e + m] = N.Matrix(_ptr(d), _ptr(s))
        shared = None
        if spec.shared_intermediate:
            shared = (N.Matrix * 3)()
            for m in range(3):
                d, s = layer.shared[m]
                shared[m] = N.Matrix(_ptr(d), _ptr(s))
        self._mats, self._shared = mats, shared
        desc = N.Desc(spec.hidden, E, spec.top_k, spec.intermediate, spec.shared_intermediate,
                      spec.expert_format, spec.shared_format, spec.router, spec.composition,
                      spec.n_group, spec.topk_group, int(spec.normalize),
                      float(spec.routed_scaling_factor), max_tokens,
                      float(spec.swiglu_limit))
        # tid2eid [vocab, k] int64, in the memory the source names (checked and copied)
        table = getattr(layer, "hash_experts", None)
        self.hashed = table is not None
        if table is not None and source == N.SOURCE_HOST:
            table = np.ascontiguousarray(table, dtype=np.int64)
        w = N.Weights(_ptr(layer.router_weight), _ptr(layer.correction_bias),
                      ctypes.addressof(mats), None if shared is None else ctypes.addressof(shared),
                      _ptr(getattr(layer, "shared_expert_gate", None)), _ptr(table),
                      0 if table is None else int(table.shape[0]))
        ctx = ctypes.c_void_p()
        st = lib.urb_moe_create(ctypes.byref(desc), ctypes.byref(w), source, ctypes.byref(ctx))
        N.check(st, "urb_moe_create")
        self._ctx = ctx

    # -- stream-ordered form ------------------------------------------------------------
    def forward_into(self, x, y, ids=None, weights=None, stream=None, token_ids=None) -> None:
        """``token_ids`` [T] (int32/uint32 device tensor): the tokens' ids, which a layer with a
        hash table routes by (``urb_moe_forward_tokens``)."""
        T = x.shape[0]
        if x.dtype != torch.float32 or not x.is_contiguous() or x.shape[-1] != self.spec.hidden:
            raise ValueError("x must be a contiguous float32 [T, hidden] tensor")
        if token_ids is None:
            N.check(N.moe_lib().urb_moe_forward(self._ctx, _ptr(x), T, _ptr(y), _ptr(ids),
                                                _ptr(weights), _stream_handle(stream)),
                    "urb_moe_forward")
            return
        if token_ids.numel() != T or token_ids.element_size() != 4:
            raise ValueError("token_ids must hold one 32-bit id per token")
        N.check(N.moe_lib().urb_moe_forward_tokens(self._ctx, _ptr(x), _ptr(token_ids), T,
                                                   _ptr(y), _ptr(ids), _ptr(weights),
                                                   _stream_handle(stream)),
                "urb_moe_forward_tokens")

    def sync(self, stream=None) -> None:
        N.check(N.moe_lib().urb_moe_sync(self._ctx, _stream_handle(stream)), "urb_moe_sync")

    # -- Result-shaped form (the reference's call signature) ---------------------------
    def forward(self, x: "torch.Tensor", token_ids: Optional["torch.Tensor"] = None):
        """x [T, H] f32 on the device -> (y [T, H], ids [T, k], weights [T, k]); raises
        UrbError like the reference's Err.  ``token_ids`` [T]: see ``forward_into``."""
        T = x.shape[0]
        y = torch.empty((T, self.spec.hidden), dtype=torch.float32, device=x.device)
        ids = torch.empty((T, self.spec.top_k), dtype=torch.int32, device=x.device)
        w = torch.empty((T, self.spec.top_k), dtype=torch.float32, device=x.device)
        self.forward_into(x, y, ids, w, token_ids=token_ids)
        self.sync()
        return y, ids, w

    def forward_block(self, h: "torch.Tensor", norm_weight: "torch.Tensor", eps: float):
        """The Qwen3.6 decoder layer's FFN block around this MoE layer (``urb_moe_forward_block``):
        h [T, H] residual stream -> (bf16(h + moe(bf16(rmsnorm(h)))), ids, weights)."""
        T = h.shape[0]
        out = torch.empty((T, self.spec.hidden), dtype=torch.float32, device=h.device)
        ids = torch.empty((T, self.spec.top_k), dtype=torch.int32, device=h.device)
        w = torch.empty((T, self.spec.top_k), dtype=torch.float32, device=h.device)
        N.check(N.moe_lib().urb_moe_forward_block(self._ctx, _ptr(h), _ptr(norm_weight),
                                                  float(eps), T, _ptr(out), _ptr(ids), _ptr(w),
                                                  _stream_handle()), "urb_moe_forward_block")
        self.sync()
        return out, ids, w

    def route(self, x: "torch.Tensor", token_ids: Optional["torch.Tensor"] = None):
        T = x.shape[0]
        logits = torch.empty((T, self.spec.n_experts), dtype=torch.float32, device=x.device)
        ids = torch.empty((T, self.spec.top_k), dtype=torch.int32, device=x.device)
        w = torch.empty((T, self.spec.top_k), dtype=torch.float32, device=x.device)
        if token_ids is None:
            N.check(N.moe_lib().urb_moe_route(self._ctx, _ptr(x), T, _ptr(logits), _ptr(ids),
                                              _ptr(w), _stream_handle()), "urb_moe_route")
        else:
            N.check(N.moe_lib().urb_moe_route_tokens(self._ctx, _ptr(x), _ptr(token_ids), T,
                                                     _ptr(logits), _ptr(ids), _ptr(w),
                                                     _stream_handle()), "urb_moe_route_tokens")
        self.sync()
        return logits, ids, w

    def profile(self, enable: bool) -> None:
        N.check(N.moe_lib().urb_moe_profile(self._ctx, int(enable)), "urb_moe_profile")

    def profile_read(self):
        """{stage: (total_ms, launches)} since profiling was enabled."""
        ms = (ctypes.c_double * len(N.STAGES))()
        calls = (ctypes.c_uint64 * len(N.STAGES))()
        N.check(N.moe_lib().urb_moe_profile_read(self._ctx, ms, calls), "urb_moe_profile_read")
        return {name: (ms[i], calls[i]) for i, name in enumerate(N.STAGES)}

    def memory(self):
        wb, ws = ctypes.c_size_t(), ctypes.c_size_t()
        N.check(N.moe_lib().urb_moe_memory(self._ctx, ctypes.byref(wb), ctypes.byref(ws)))
        return wb.value, ws.value

    def close(self) -> None:
        if getattr(self, "_ctx", None):
            N.moe_lib().urb_moe_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def expert_views(fmt: int, n_experts: int, hidden: int, intermediate: int, gate_up,
                 gate_up_scales, down, down_scales) -> List[Tuple[int, Optional[int]]]:
    """``urb_expert_views``: (data, scales) addresses of every expert's gate, up and down
    inside consolidated tensors, in urb_moe_weights.experts order."""
    out = (N.Matrix * (3 * n_experts))()
    N.check(N.moe_lib().urb_expert_views(fmt, n_experts, hidden, intermediate, _ptr(gate_up),
                                         _ptr(gate_up_scales), _ptr(down), _ptr(down_scales),
                                         ctypes.addressof(out)), "urb_expert_views")
    return [(m.data, m.scales) for m in out]


def pack_matrix(fmt: int, data, scales, rows: int, cols: int):
    """Row-major device matrix -> (data, scales) in the panel layout the context streams."""
    pd = torch.empty_like(data)
    ps = None if scales is None else torch.empty_like(scales)
    N.check(N.moe_lib().urb_pack_matrix(fmt, _ptr(data), _ptr(scales), rows, cols, _ptr(pd),
                                        _ptr(ps), _stream_handle()), "urb_pack_matrix")
    return pd, ps


def zc_rms_norm_bf16(x, weight, eps: float):
    """``urb_zc_rms_norm_bf16``: bf16(zero_centered_rms_norm(x, weight, eps)) of x [rows, H]."""
    out = torch.empty_like(x)
    N.check(N.moe_lib().urb_zc_rms_norm_bf16(_ptr(x), _ptr(weight), x.shape[0], x.shape[1],
                                             float(eps), _ptr(out), _stream_handle()),
            "urb_zc_rms_norm_bf16")
    torch.cuda.synchronize()
    return out


def quantize_e4m3(x, block: int = 32):
    """simulate_e4m3_activation of a [rows, cols] f32 device tensor as (E4M3 codes, E8M0
    scales) device tensors, blocks of ``block`` (32 or 128) values along each row."""
    if x.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError("quantize_e4m3 takes a contiguous float32 tensor")
    rows, cols = x.shape
    codes = torch.empty((rows, cols), dtype=torch.uint8, device=x.device)
    scales = torch.empty((rows, cols // block), dtype=torch.uint8, device=x.device)
    N.check(N.moe_lib().urb_quantize_e4m3_blocks(_ptr(x), rows, cols, block, _ptr(codes),
                                                 _ptr(scales), _stream_handle()),
            "urb_quantize_e4m3_blocks")
    return codes, scales


def packed_layer(layer: "DeviceLayer") -> "DeviceLayer":
    """The same layer with every expert and shared matrix converted to the panel layout, for
    URB_SOURCE_DEVICE_BORROW."""
    spec = layer.spec
    H, I, Is = spec.hidden, spec.intermediate, spec.shared_intermediate
    dims = ((I, H), (I, H), (H, I))
    sdims = ((Is, H), (Is, H), (H, Is))
    ex = [[pack_matrix(spec.expert_format, d, sc, *dims[m]) for m, (d, sc) in enumerate(trip)]
          for trip in layer.experts]
    sh = None
    if layer.shared is not None:
        sh = [pack_matrix(spec.shared_format, d, sc, *sdims[m])
              for m, (d, sc) in enumerate(layer.shared)]
    torch.cuda.current_stream().synchronize()
    return DeviceLayer(spec, layer.router_weight, ex, sh, layer.correction_bias, None,
                       layer.shared_expert_gate, layer.hash_experts)


def dequant_rows(fmt: int, data, scales, rows: int, cols: int, row0: int = 0,
                 count: Optional[int] = None) -> "torch.Tensor":
    """Dequantised rows of a device matrix (MxFp4Matrix::row and friends), bit-exact."""
    count = rows - row0 if count is None else count
    out = torch.empty((count, cols), dtype=torch.float32, device=data.device)
    N.check(N.moe_lib().urb_dequant_rows(fmt, _ptr(data), _ptr(scales), rows, cols, row0, count,
                                         _ptr(out), _stream_handle()), "urb_dequant_rows")
    torch.cuda.current_stream().synchronize()
    return out


def synth_activations(tokens: int, hidden: int, name: str = "x",
                      base_seed: int = synth.BASE_SEED, device="cuda") -> "torch.Tensor":
    x = torch.empty((tokens, hidden), dtype=torch.float32, device=device)
    N.check(N.synth_lib().urb_synth_activations(synth.stream_seed(name, base_seed),
                                                tokens * hidden, x.data_ptr(),
                                                _stream_handle()), "synth activations")
    return x
