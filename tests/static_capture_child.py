"""Child process of test_zz_no_alloc.test_first_static_call_under_capture:
its FIRST lrmoe_moe_layer_static call is made while the stream captures a
HIP graph.  Checks that the captured graph holds exactly one node (the
decode kernel: no scratch clear was recorded), and that replays, interleaved
with eager static calls and workspace calls, give outputs, routes and
routing weights bit-identical to lrmoe_moe_layer with a workspace.  Prints
"static capture ok" and exits 0 on success."""

from __future__ import annotations

import ctypes as C
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

from lightreason_amd import _native  # noqa: E402
from lightreason_amd.moe import Workspace, moe_layer  # noqa: E402
from lightreason_amd.synthetic import SyntheticModel  # noqa: E402


def _ptr(t):
    return None if t is None else t.data_ptr()


def main() -> int:
    device = torch.device("cuda:0")
    _native.device_check()
    lib = _native.library()
    model = SyntheticModel(layers=1, device=device, seed=515, shared=True, norm="normal")
    layer = model.layers[0]
    T = 4
    x = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
    out = torch.empty_like(x)
    idx = torch.empty((T, 8), dtype=torch.int64, device=device)
    wts = torch.empty((T, 8), dtype=torch.bfloat16, device=device)
    status = torch.zeros((1,), dtype=torch.int32, device=device)
    ws = Workspace(device, T)

    def static_call(stream):
        return lib.lrmoe_moe_layer_static(
            _ptr(x), T, _ptr(layer.router), None, _ptr(layer.expert_ptrs), None, _ptr(layer.shared_gate_proj),
            _ptr(layer.shared_up_proj), _ptr(layer.shared_down_proj), _ptr(layer.shared_expert_gate),
            _ptr(layer.norm_weight), C.c_float(layer.eps), _ptr(out), _ptr(idx), _ptr(wts), _ptr(status), stream)

    def check(tag):
        torch.cuda.synchronize()
        want_i = torch.empty_like(idx)
        want_w = torch.empty_like(wts)
        want = moe_layer(x, layer, indices=want_i, weights=want_w, workspace=ws)
        torch.cuda.synchronize()
        assert ws.status() == 0 and int(status.item()) == 0, tag
        assert torch.equal(idx, want_i), tag
        assert torch.equal(wts.view(torch.int16), want_w.view(torch.int16)), tag
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), tag
        print(f"[static capture] {tag}: bit-identical", flush=True)

    x.copy_(model.hidden(T, step=1))
    moe_layer(x, layer, workspace=ws)      # the library is loaded and warm; no static call yet
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph(keep_graph=True)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            rc = static_call(torch.cuda.current_stream(device).cuda_stream)
    torch.cuda.current_stream(device).wait_stream(stream)
    assert rc == 0, f"captured static call returned {rc}"
    hip = C.CDLL("libamdhip64.so")
    nodes = C.c_size_t(0)
    err = hip.hipGraphGetNodes(C.c_void_p(graph.raw_cuda_graph()), None, C.byref(nodes))
    assert err == 0, f"hipGraphGetNodes: {err}"
    print(f"[static capture] captured graph nodes: {nodes.value}", flush=True)
    assert nodes.value == 1, "the first static call under capture recorded more than its decode kernel"
    graph.instantiate()
    for rep in range(4):
        x.copy_(model.hidden(T, step=10 + rep))
        graph.replay()
        check(f"replay {rep}")
        x.copy_(model.hidden(T, step=100 + rep))
        assert static_call(torch.cuda.current_stream(device).cuda_stream) == 0
        check(f"eager static call {rep}")
    print("static capture ok", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
