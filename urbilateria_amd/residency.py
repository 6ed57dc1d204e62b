"""The HBM expert-residency policy (``include/urb_residency.h``): LayerLruCache's deterministic
per-layer LRU (src/runtime/cache.rs:66-519) behind the C ABI, mirrored with the reference's
method names.  Values are 64-bit handles (an HBM slot, a device pointer) the caller owns; loads
are Python callables returning ``(value, resident_bytes, read_bytes)`` or raising."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Callable, List, Optional, Sequence, Tuple

from . import native as N

Load = Callable[[], Tuple[int, int, int]]


class Telemetry(ctypes.Structure):
    """ExpertTelemetry (src/runtime/cache.rs:5-28)."""
    _fields_ = [("hits", ctypes.c_uint64), ("misses", ctypes.c_uint64),
                ("evictions", ctypes.c_uint64), ("bytes_read", ctypes.c_uint64),
                ("resident_experts", ctypes.c_uint64), ("resident_bytes", ctypes.c_uint64)]

    def accesses(self) -> int:
        return self.hits + self.misses

    def hit_rate(self) -> Optional[float]:
        a = self.accesses()
        return None if a == 0 else self.hits / a

    def as_tuple(self):
        return (self.hits, self.misses, self.evictions, self.bytes_read, self.resident_experts,
                self.resident_bytes)

    def copy(self) -> "Telemetry":
        t = Telemetry()
        ctypes.pointer(t)[0] = self
        return t

    def __eq__(self, other) -> bool:
        return isinstance(other, Telemetry) and self.as_tuple() == other.as_tuple()


LOAD_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64,
                           ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                           ctypes.POINTER(ctypes.c_uint64))


class LoadError(RuntimeError):
    """A load callable raised; the access returned its error without admitting the key.
    ``evicted`` is the handle a plain access displaced before loading (the caller releases it),
    or None."""

    evicted: Optional[int] = None


_U64 = ctypes.c_uint64


def _keys(keys: Sequence[int]):
    return (_U64 * max(len(keys), 1))(*keys)


def _bind(lib) -> None:
    if getattr(lib, "_urb_lru_bound", False):
        return
    P, u32, u64, sz = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_size_t
    pu64, pint, psz = ctypes.POINTER(u64), ctypes.POINTER(ctypes.c_int), ctypes.POINTER(sz)
    sig = {
        "urb_lru_create": ([u32, P, ctypes.POINTER(P)], ctypes.c_int),
        "urb_lru_destroy": ([P], None),
        "urb_lru_access": ([P, P, u32, u64, LOAD_FN, P, pu64, pu64, pint], ctypes.c_int),
        "urb_lru_contains": ([P, u32, u64], ctypes.c_int),
        "urb_lru_peek": ([P, u32, u64, pu64], ctypes.c_int),
        "urb_lru_layer_is_empty": ([P, u32], ctypes.c_int),
        "urb_lru_layer_capacity": ([P, u32], u32),
        "urb_lru_residency": ([P, u32, pu64, pu64], None),
        "urb_lru_entries": ([P, u32, P, P, P], sz),
        "urb_lru_clock": ([P], u64),
        "urb_lru_set_clock": ([P, u64], None),
        "urb_lru_drain_layer": ([P, P, u32, P], sz),
        "urb_lru_can_insert_without_eviction": ([P, u32, P, sz], ctypes.c_int),
        "urb_lru_projected_misses": ([P, u32, P, sz], sz),
        "urb_lru_grouped_access_order": ([P, u32, P, sz, P, psz], ctypes.c_int),
        "urb_lru_finish_grouped_accesses": ([P, u32, P, sz, sz], None),
        "urb_lru_grouped_access_plan": ([P, u32, P, sz], P),
        "urb_lru_plan_destroy": ([P], None),
        "urb_lru_plan_order": ([P, P], sz),
        "urb_lru_access_grouped": ([P, P, P, u64, LOAD_FN, P, pu64, pu64, pint], ctypes.c_int),
        "urb_lru_finish_grouped_plan": ([P, P], None),
        "urb_lru_prepare_ordered_batch": ([P, P, u32, P, sz, P, psz], ctypes.c_int),
        "urb_lru_lend_unused_capacity": ([P, u32, u32], u32),
        "urb_lru_restore_layer_capacity": ([P, P, u32, u32, P], sz),
    }
    for name, (args, res) in sig.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = res
    lib._urb_lru_bound = True


EXPORTS = ("urb_lru_create", "urb_lru_destroy", "urb_lru_access", "urb_lru_contains",
           "urb_lru_peek", "urb_lru_layer_is_empty", "urb_lru_layer_capacity",
           "urb_lru_residency", "urb_lru_entries", "urb_lru_clock", "urb_lru_set_clock",
           "urb_lru_drain_layer", "urb_lru_can_insert_without_eviction",
           "urb_lru_projected_misses", "urb_lru_grouped_access_order",
           "urb_lru_finish_grouped_accesses", "urb_lru_grouped_access_plan",
           "urb_lru_plan_destroy", "urb_lru_plan_order", "urb_lru_access_grouped",
           "urb_lru_finish_grouped_plan", "urb_lru_prepare_ordered_batch",
           "urb_lru_lend_unused_capacity", "urb_lru_restore_layer_capacity")


@dataclass
class Entry:
    key: int
    last_used: int
    value: int


class GroupedAccessPlan:
    """GroupedAccessPlan (src/runtime/cache.rs:38-64)."""

    def __init__(self, lib, handle: int, layer: int, n: int):
        self._lib, self._h, self.layer = lib, handle, layer
        buf = (_U64 * max(n, 1))()
        m = lib.urb_lru_plan_order(handle, buf)
        self._order = [buf[i] for i in range(m)]

    def order(self) -> List[int]:
        return list(self._order)

    def __del__(self):
        if getattr(self, "_h", None):
            self._lib.urb_lru_plan_destroy(self._h)
            self._h = None


class LayerLruCache:
    """LayerLruCache<T> (src/runtime/cache.rs:66-519) over 64-bit handles."""

    def __init__(self, layers: int, slots_per_layer: int = 0,
                 layer_capacities: Optional[Sequence[int]] = None):
        self._lib = N.moe_lib()
        _bind(self._lib)
        caps = list(layer_capacities) if layer_capacities is not None else \
            [slots_per_layer] * layers
        arr = (ctypes.c_uint32 * max(len(caps), 1))(*caps)
        h = ctypes.c_void_p()
        N.check(self._lib.urb_lru_create(len(caps), arr, ctypes.byref(h)), "urb_lru_create")
        self._h = h
        self._caps = len(caps)
        self._error: Optional[BaseException] = None

    @staticmethod
    def with_layer_capacities(capacities: Sequence[int]) -> "LayerLruCache":
        return LayerLruCache(len(capacities), layer_capacities=capacities)

    def close(self) -> None:
        if self._h:
            self._lib.urb_lru_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    # -- loads ------------------------------------------------------------------------------
    def _callback(self, load: Load):
        def fn(_user, _layer, _key, value, nbytes, read):
            try:
                v, b, r = load()
            except BaseException as e:  # handed back through the access's return code
                self._error = e
                return 1
            value[0], nbytes[0], read[0] = v, b, r
            return 0
        return LOAD_FN(fn)

    def _finish(self, st: int, cb, evicted: Optional[int] = None) -> None:
        del cb
        if st:
            err, self._error = self._error, None
            e = LoadError("load failed")
            e.evicted = evicted
            raise e from err

    # -- accesses ----------------------------------------------------------------------------
    def access_with_evicted(self, telemetry: Telemetry, layer: int, key: int,
                            load: Load) -> Tuple[int, Optional[int]]:
        """(resident or loaded value, displaced value or None)."""
        v, e, he = _U64(), _U64(), ctypes.c_int()
        cb = self._callback(load)
        st = self._lib.urb_lru_access(self._h, ctypes.byref(telemetry), layer, key, cb, None,
                                      ctypes.byref(v), ctypes.byref(e), ctypes.byref(he))
        self._finish(st, cb, e.value if he.value else None)
        return v.value, (e.value if he.value else None)

    def access(self, telemetry: Telemetry, layer: int, key: int, load: Load) -> int:
        return self.access_with_evicted(telemetry, layer, key, load)[0]

    def contains(self, layer: int, key: int) -> bool:
        return bool(self._lib.urb_lru_contains(self._h, layer, key))

    def peek(self, layer: int, key: int) -> Optional[int]:
        v = _U64()
        return v.value if self._lib.urb_lru_peek(self._h, layer, key, ctypes.byref(v)) else None

    def layer_is_empty(self, layer: int) -> bool:
        return bool(self._lib.urb_lru_layer_is_empty(self._h, layer))

    def layer_capacity(self, layer: int) -> int:
        return self._lib.urb_lru_layer_capacity(self._h, layer)

    def residency(self) -> List[Tuple[int, int, int, int]]:
        """[(layer, experts, capacity, bytes)] (src/runtime/cache.rs:75-89)."""
        out = []
        for layer in range(self._caps):
            e, b = _U64(), _U64()
            self._lib.urb_lru_residency(self._h, layer, ctypes.byref(e), ctypes.byref(b))
            out.append((layer, e.value, self.layer_capacity(layer), b.value))
        return out

    def entries(self, layer: int) -> List[Entry]:
        n = max(self.layer_capacity(layer), 1) + 64
        k, u, v = (_U64 * n)(), (_U64 * n)(), (_U64 * n)()
        m = self._lib.urb_lru_entries(self._h, layer, k, u, v)
        return [Entry(k[i], u[i], v[i]) for i in range(m)]

    @property
    def clock(self) -> int:
        return self._lib.urb_lru_clock(self._h)

    @clock.setter
    def clock(self, value: int) -> None:
        self._lib.urb_lru_set_clock(self._h, value)

    def drain_layer(self, telemetry: Telemetry, layer: int) -> List[int]:
        n = len(self.entries(layer))
        out = (_U64 * max(n, 1))()
        m = self._lib.urb_lru_drain_layer(self._h, ctypes.byref(telemetry), layer, out)
        return [out[i] for i in range(m)]

    def can_insert_without_eviction(self, layer: int, keys: Sequence[int]) -> bool:
        return bool(self._lib.urb_lru_can_insert_without_eviction(self._h, layer, _keys(keys),
                                                                  len(keys)))

    def projected_misses(self, layer: int, keys: Sequence[int]) -> int:
        return self._lib.urb_lru_projected_misses(self._h, layer, _keys(keys), len(keys))

    def grouped_access_order(self, layer: int, keys: Sequence[int]) -> Optional[List[int]]:
        out = (_U64 * max(len(keys), 1))()
        n = ctypes.c_size_t()
        if not self._lib.urb_lru_grouped_access_order(self._h, layer, _keys(keys), len(keys), out,
                                                      ctypes.byref(n)):
            return None
        return [out[i] for i in range(n.value)]

    def finish_grouped_accesses(self, layer: int, keys: Sequence[int], groups: int) -> None:
        self._lib.urb_lru_finish_grouped_accesses(self._h, layer, _keys(keys), len(keys), groups)

    def grouped_access_plan(self, layer: int, keys: Sequence[int]) -> Optional[GroupedAccessPlan]:
        h = self._lib.urb_lru_grouped_access_plan(self._h, layer, _keys(keys), len(keys))
        return None if not h else GroupedAccessPlan(self._lib, h, layer, len(keys))

    def access_grouped_with_evicted(self, telemetry: Telemetry, plan: GroupedAccessPlan,
                                    key: int, load: Load) -> Tuple[int, Optional[int]]:
        v, e, he = _U64(), _U64(), ctypes.c_int()
        cb = self._callback(load)
        st = self._lib.urb_lru_access_grouped(self._h, ctypes.byref(telemetry), plan._h, key, cb,
                                              None, ctypes.byref(v), ctypes.byref(e),
                                              ctypes.byref(he))
        self._finish(st, cb)
        return v.value, (e.value if he.value else None)

    def finish_grouped_plan(self, plan: GroupedAccessPlan) -> None:
        self._lib.urb_lru_finish_grouped_plan(self._h, plan._h)

    def prepare_ordered_batch(self, telemetry: Telemetry, layer: int,
                              keys: Sequence[int]) -> Optional[List[int]]:
        out = (_U64 * max(len(keys), 1))()
        n = ctypes.c_size_t()
        if not self._lib.urb_lru_prepare_ordered_batch(self._h, ctypes.byref(telemetry), layer,
                                                       _keys(keys), len(keys), out,
                                                       ctypes.byref(n)):
            return None
        return [out[i] for i in range(n.value)]

    def lend_unused_capacity(self, layer: int, maximum: int) -> int:
        return self._lib.urb_lru_lend_unused_capacity(self._h, layer, maximum)

    def restore_layer_capacity(self, telemetry: Telemetry, layer: int,
                               capacity: int) -> List[int]:
        n = len(self.entries(layer))
        out = (_U64 * max(n, 1))()
        m = self._lib.urb_lru_restore_layer_capacity(self._h, ctypes.byref(telemetry), layer,
                                                     capacity, out)
        return [out[i] for i in range(m)]


def _to_device(a):
    """Device copy of a host array or CPU tensor (bytes preserved); device tensors pass."""
    import numpy as np
    import torch
    if a is None or (isinstance(a, torch.Tensor) and a.is_cuda):
        return a
    if isinstance(a, torch.Tensor):
        a = a.numpy()
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


class StreamedMoeLayer:
    """A layer whose experts stay in caller memory (the reference's expert store), with at most
    ``slots`` of them resident in HBM at a time, placed by the residency policy.

    A call routes first (``urb_moe_route``), replays the batch's expert accesses in the
    reference's order -- each token's experts in ascending id, tokens in order, as
    execute_batched_moe builds them (src/models/qwen3_6/runtime.rs:1086-1104) -- through the
    LRU, packing each miss into the slot its victim frees (``urb_pack_matrix``) and repointing
    the context's table (``urb_moe_set_expert``), then runs the layer.  A batch needing more
    distinct experts than slots is cut into token runs that fit."""

    def __init__(self, layer, slots: int, max_tokens: int, layer_index: int = 0,
                 cache: Optional[LayerLruCache] = None):
        import torch
        from . import configs as C
        from . import moe
        spec = layer.spec
        if slots < spec.top_k:
            raise ValueError("a token's experts must fit the slots at once")
        self.spec, self.slots, self.layer_index = spec, slots, layer_index
        self._src = layer
        H, I = spec.hidden, spec.intermediate
        self._dims = ((I, H), (I, H), (H, I))
        sizes = [C.matrix_bytes(spec.expert_format, r, c) for r, c in self._dims]
        al = lambda n: (n + 255) // 256 * 256
        self._slot_bytes = sum(al(d) + al(s) for d, s in sizes)
        self._arena = torch.empty(slots * self._slot_bytes, dtype=torch.uint8, device="cuda")
        self._slot_mats = []
        for k in range(slots):
            off, mats = k * self._slot_bytes, []
            for d, s in sizes:
                data = self._arena[off:off + d]
                off += al(d)
                sc = self._arena[off:off + s] if s else None
                off += al(s)
                mats.append((data, sc))
            self._slot_mats.append(mats)
        self._pack(0, 0)  # every table entry starts at slot 0, which holds valid matrices
        shared = None
        if layer.shared is not None:  # always resident, in the panel layout too
            Is = spec.shared_intermediate
            sdims = ((Is, H), (Is, H), (H, Is))
            shared = [moe.pack_matrix(spec.shared_format, _to_device(d), _to_device(sc),
                                      *sdims[m])
                      for m, (d, sc) in enumerate(layer.shared)]
        torch.cuda.synchronize()
        placeholder = moe.DeviceLayer(spec, _to_device(layer.router_weight),
                                      [self._slot_mats[0]] * spec.n_experts, shared,
                                      _to_device(layer.correction_bias), None,
                                      _to_device(getattr(layer, "shared_expert_gate", None)),
                                      _to_device(getattr(layer, "hash_experts", None)))
        self.layer = moe.MoeLayer(placeholder, max_tokens, source=N.SOURCE_DEVICE_BORROW)
        self.cache = cache if cache is not None else LayerLruCache(layer_index + 1, slots)
        self._check_capacity()
        self.telemetry = Telemetry()

    def _check_capacity(self) -> None:
        # one slot per resident expert: a layer capacity other than `slots` (another cache, or
        # capacity lent by lend_unused_capacity) would admit experts with no slot to hold them
        cap = self.cache.layer_capacity(self.layer_index)
        if cap != self.slots:
            raise ValueError(f"the cache holds {cap} experts of layer {self.layer_index}, the "
                             f"layer has {self.slots} HBM slots")

    def _free_slot(self) -> int:
        """A slot no resident expert of the layer holds.  Called from the load, after the access
        evicted its victim, so the cache's own entries say which slots are in use."""
        used = {e.value for e in self.cache.entries(self.layer_index)}
        for slot in range(self.slots):
            if slot not in used:
                return slot
        raise RuntimeError("no free HBM slot although the cache has room")

    def _pack(self, expert: int, slot: int) -> None:
        from . import moe

        for m, (r, c) in enumerate(self._dims):
            # host sources (numpy, CPU tensors) are staged on the device first
            d, s = (_to_device(a) for a in self._src.experts[expert][m])
            pd, ps = self._slot_mats[slot][m]
            N.check(N.moe_lib().urb_pack_matrix(self.spec.expert_format, moe._ptr(d), moe._ptr(s),
                                                r, c, moe._ptr(pd), moe._ptr(ps),
                                                moe._stream_handle()), "urb_pack_matrix")

    def _point(self, expert: int, slot: int) -> None:
        from . import moe
        mats = (N.Matrix * 3)(*[N.Matrix(moe._ptr(d), moe._ptr(s))
                                for d, s in self._slot_mats[slot]])
        N.check(N.moe_lib().urb_moe_set_expert(self.layer._ctx, expert, ctypes.addressof(mats),
                                               moe._stream_handle()), "urb_moe_set_expert")

    def _access(self, key: int) -> None:
        """One expert access through the policy.  A miss packs the expert into a free slot (never
        one a resident expert uses) and repoints the table after validating it; a failed load
        (bad payload, pack error) leaves every resident expert and its slot untouched, and the
        slot it wrote stays free, so later calls are unaffected."""
        def load(key=key):
            slot = self._free_slot()
            self._pack(key, slot)
            self._point(key, slot)
            return slot, self._slot_bytes, self._slot_bytes
        self.cache.access_with_evicted(self.telemetry, self.layer_index, key, load)

    def forward(self, x, token_ids=None):
        """x [T, H] f32 (device) -> (y, ids, weights) of the resident layer; ``token_ids`` [T]
        for a layer with a hash table."""
        import torch
        self._check_capacity()
        T = x.shape[0]
        _, ids, _ = self.layer.route(x, token_ids=token_ids)
        ids = ids.cpu().tolist()
        runs, start, seen = [], 0, set()
        for t in range(T):
            nxt = seen | set(ids[t])
            if len(nxt) > self.slots:
                runs.append((start, t))
                start, nxt = t, set(ids[t])
            seen = nxt
        runs.append((start, T))
        self.last_runs = runs
        ys, idl, wl = [], [], []
        for a, b in runs:
            for t in range(a, b):
                for key in sorted(ids[t]):
                    self._access(key)
            y, i, w = self.layer.forward(
                x[a:b].contiguous(), token_ids=None if token_ids is None else token_ids[a:b])
            ys.append(y)
            idl.append(i)
            wl.append(w)
        return torch.cat(ys), torch.cat(idl), torch.cat(wl)

    def close(self) -> None:
        self.layer.close()
