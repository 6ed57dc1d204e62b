"""The allocation-free layer call (urb_moe_forward_noalloc) through the C ABI: on the same layer
and inputs it gives urb_moe_forward's outputs, expert ids and route weights bit for bit, on two
calls in a row (the second smaller, so stale scratch contents from the first would show), and it
refuses calls whose buffers exceed its scratch."""

import ctypes

import numpy as np
import pytest

from urbilateria_amd import configs as C
from urbilateria_amd import native as N
from urbilateria_amd import synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu(require_gpu):
    from urbilateria_amd import moe  # noqa: F401  (fails loudly without liburb_moe.so)
    torch.cuda.set_device(0)
    yield


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _call(fn, layer, x):
    T = x.shape[0]
    y = torch.full((T, layer.spec.hidden), float("nan"), dtype=torch.float32, device="cuda")
    ids = torch.full((T, layer.spec.top_k), -1, dtype=torch.int32, device="cuda")
    w = torch.full((T, layer.spec.top_k), float("nan"), dtype=torch.float32, device="cuda")
    N.check(fn(layer._ctx, _p(x), T, _p(y), _p(ids), _p(w), None), fn.__name__)
    layer.sync()
    return y, ids, w


def _layers():
    from urbilateria_amd import moe
    out = []
    for name in ("c1_bf16_decode", "c3_mxfp4_decode", "c4_mxfp8", "c5_mxfp4_dsv41"):
        w = C.workload(name)
        spec = C.small_spec(w.spec, hidden=256, n_experts=16, intermediate=128)
        bias = C.zipf_bias(spec.n_experts, w.zipf_s, 0.05) if w.zipf_s else None
        out.append((name, moe.MoeLayer(C.make_host_layer(spec, bias=bias), max_tokens=64)))
    return out


@pytest.mark.parametrize("shape", ["small", "c3_full"])
def test_noalloc_forward_equals_forward_on_two_calls(shape):
    from urbilateria_amd import moe
    lib = N.moe_lib()
    if shape == "small":
        layers = _layers()
        sizes = (40, 3)
    else:
        spec = C.workload("c3_mxfp4_decode").spec
        layers = [("c3_mxfp4_decode", moe.MoeLayer(moe.DeviceLayer.synthesize(spec),
                                                   max_tokens=8))]
        sizes = (8, 1)
    for name, layer in layers:
        for call, T in enumerate(sizes):
            x = torch.from_numpy(synth.activations(f"x.noalloc.{name}.{call}", T,
                                                   layer.spec.hidden)).cuda()
            ref = _call(lib.urb_moe_forward, layer, x)
            got = _call(lib.urb_moe_forward_noalloc, layer, x)
            for a, b in zip(got, ref):
                assert torch.equal(a, b), (name, T)
        layer.close()


def test_noalloc_forward_refuses_what_its_scratch_cannot_hold():
    from urbilateria_amd import moe
    lib = N.moe_lib()
    spec = C.workload("c5_mxfp4_zipf_prefill").spec
    layer = moe.MoeLayer(moe.DeviceLayer.synthesize(spec), max_tokens=1024)
    # a zero batch routes by ties to the lowest ids; the documented capacity of this shape is 88
    x = torch.zeros((1024, spec.hidden), dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for T, want in ((1024, N.ERR_SHAPE), (0, N.ERR_SHAPE), (89, N.ERR_SHAPE), (88, N.OK),
                    (1, N.OK)):
        st = lib.urb_moe_forward_noalloc(layer._ctx, _p(x), T, _p(y), None, None, None)
        assert st == want, T
    layer.sync()
    layer.close()
