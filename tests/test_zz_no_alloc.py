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


def _small(name, max_tokens=64):
    from urbilateria_amd import moe
    w = C.workload(name)
    spec = C.small_spec(w.spec, hidden=256, n_experts=16, intermediate=128)
    bias = C.zipf_bias(spec.n_experts, w.zipf_s, 0.05) if w.zipf_s else None
    return moe.MoeLayer(C.make_host_layer(spec, bias=bias), max_tokens=max_tokens)


def _layers():
    # qwen36_release: the QWEN36 composition with its gated shared expert, whose gate logits
    # are carved from the scratch too
    return [(name, _small(name)) for name in ("c1_bf16_decode", "c3_mxfp4_decode", "c4_mxfp8",
                                              "c5_mxfp4_dsv41", "qwen36_release")]


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


def test_noalloc_batch_with_routing_beside_the_shared_expert():
    # 300 tokens of a GLM layer with a shared expert (f32 activations): the shared expert runs in
    # line and the router, routing and permutation on the layer's side stream, all of their
    # buffers in the scratch
    lib = N.moe_lib()
    layer = _small("c3_mxfp4_decode", max_tokens=320)
    for call, T in enumerate((300, 257)):
        x = torch.from_numpy(synth.activations(f"x.noalloc.beside.{call}", T,
                                               layer.spec.hidden)).cuda()
        ref = _call(lib.urb_moe_forward, layer, x)
        got = _call(lib.urb_moe_forward_noalloc, layer, x)
        for a, b in zip(got, ref):
            assert torch.equal(a, b), T
    layer.close()


def test_noalloc_refuses_hash_routed_layers():
    from urbilateria_amd import moe
    lib = N.moe_lib()
    w = C.workload("dsv4_flash_hash")
    spec = C.small_spec(w.spec, hidden=256, n_experts=32, intermediate=128)
    host = C.make_host_layer(spec, hash_vocab=50)
    layer = moe.MoeLayer(host, max_tokens=8)
    x = torch.zeros((4, spec.hidden), dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    assert lib.urb_moe_forward_noalloc(layer._ctx, _p(x), 4, _p(y), None, None,
                                       None) == N.ERR_ARGUMENT
    layer.close()


@pytest.mark.parametrize("name,T", [("c1_bf16_decode", 40), ("c3_mxfp4_decode", 1),
                                    ("c3_mxfp4_decode", 40)])
def test_noalloc_forward_replays_under_graph_capture(name, T):
    # One warm-up call (it resolves the scratch's device address), then a call captured into a
    # graph on a side stream and replayed three times, with eager work on the outputs between
    # the replays: every replay gives urb_moe_forward's outputs bit for bit.  c3 at 40 tokens
    # forks its shared expert onto the layer's own side stream inside the capture.
    lib = N.moe_lib()
    layer = _small(name)
    x = torch.from_numpy(synth.activations(f"x.noalloc.graph.{name}.{T}", T,
                                           layer.spec.hidden)).cuda()
    ref = _call(lib.urb_moe_forward, layer, x)
    _call(lib.urb_moe_forward_noalloc, layer, x)
    y = torch.empty((T, layer.spec.hidden), dtype=torch.float32, device="cuda")
    ids = torch.empty((T, layer.spec.top_k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, layer.spec.top_k), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        st = lib.urb_moe_forward_noalloc(layer._ctx, _p(x), T, _p(y), _p(ids), _p(w),
                                         ctypes.c_void_p(stream.cuda_stream))
    assert st == N.OK
    for rep in range(3):
        y.fill_(float("nan"))
        ids.fill_(-1)
        w.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        layer.sync()
        for a, b in zip((y, ids, w), ref):
            assert torch.equal(a, b), (name, T, rep)
    del graph
    layer.close()
