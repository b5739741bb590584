"""The no-allocation decode layer (lrmoe_moe_layer_static: its scratch is a
static device array of the library) against lrmoe_moe_layer with a
workspace, through the C ABI, on an MI355X.

Bar: bit-identical outputs, routes and routing weights (both run the same
decode kernel on the same inputs), on two calls in a row with the second
smaller than the first; a clean status word; sizes beyond the maximum
rejected before any launch."""

from __future__ import annotations

import ctypes as C

import pytest
import torch

pytestmark = pytest.mark.gpu


def _ptr(t):
    return None if t is None else t.data_ptr()


def _static(lib, x, layer, out, idx, wts, status, logits=None):
    stream = torch.cuda.current_stream(x.device).cuda_stream
    return lib.lrmoe_moe_layer_static(
        _ptr(x), x.shape[0], None if logits is not None else _ptr(layer.router), _ptr(logits),
        _ptr(layer.expert_ptrs), None, _ptr(layer.shared_gate_proj), _ptr(layer.shared_up_proj),
        _ptr(layer.shared_down_proj), _ptr(layer.shared_expert_gate), _ptr(layer.norm_weight), C.c_float(layer.eps),
        _ptr(out), _ptr(idx), _ptr(wts), _ptr(status), stream)


@pytest.mark.parametrize("given_logits", [False, True])
def test_static_layer_equals_workspace_layer(model, given_logits):
    from lightreason_amd import _native
    from lightreason_amd.moe import Workspace, moe_layer

    lib = _native.library()
    layer = model.layers[0]
    device = model.device
    for i, tokens in enumerate((16, 3)):
        print(f"[no-alloc] call {i}: T={tokens} logits={'given' if given_logits else 'router'}", flush=True)
        x = model.hidden(tokens, step=9700 + 10 * i + given_logits)
        lg = (x.float() @ layer.router.float().T).to(torch.bfloat16) if given_logits else None
        ws = Workspace(device, tokens)
        idx_w = torch.empty((tokens, 8), dtype=torch.int64, device=device)
        wts_w = torch.empty((tokens, 8), dtype=torch.bfloat16, device=device)
        want = moe_layer(x, layer, indices=idx_w, weights=wts_w, logits_in=lg, workspace=ws)
        out = torch.full_like(x, float("nan"))
        idx = torch.full((tokens, 8), -7, dtype=torch.int64, device=device)
        wts = torch.zeros((tokens, 8), dtype=torch.bfloat16, device=device)
        status = torch.full((1,), -1, dtype=torch.int32, device=device)
        assert _static(lib, x, layer, out, idx, wts, status, lg) == 0
        torch.cuda.synchronize()
        assert ws.status() == 0
        assert int(status.item()) == 0
        assert torch.equal(idx, idx_w)
        assert torch.equal(wts.view(torch.int16), wts_w.view(torch.int16))
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))


def test_static_layer_rejects_oversize_and_reports_bad_routes(model):
    from lightreason_amd import _native

    lib = _native.library()
    layer = model.layers[0]
    device = model.device
    x = model.hidden(17, step=9800)
    out = torch.empty_like(x)
    assert _static(lib, x, layer, out, None, None, None) == _native.LRMOE_E_ARG
    # Without status_out the status word stays in the static scratch; a
    # call with a status word after it writes there.
    x = model.hidden(2, step=9801)
    out = torch.empty_like(x)
    assert _static(lib, x, layer, out, None, None, None) == 0
    logits = torch.zeros((2, 256), dtype=torch.bfloat16, device=device)
    status = torch.full((1,), -1, dtype=torch.int32, device=device)
    assert _static(lib, x, layer, out, None, None, status, logits) == 0
    torch.cuda.synchronize()
    assert int(status.item()) == 0   # equal logits: experts 0..7, valid routes


def test_first_static_call_under_capture(model):
    """A process whose first lrmoe_moe_layer_static call is captured into a
    graph (tests/static_capture_child.py): the graph holds only the decode
    kernel (no scratch clear recorded), and its replays, interleaved with
    eager static and workspace calls, are bit-identical to lrmoe_moe_layer.
    Run in a child process so that its static call is that process's first."""
    import subprocess
    import sys
    from pathlib import Path

    child = Path(__file__).resolve().parent / "static_capture_child.py"
    print("[no-alloc] child process: first static call under capture", flush=True)
    result = subprocess.run([sys.executable, "-u", str(child)], capture_output=True, text=True, timeout=300)
    print(result.stdout[-4000:], result.stderr[-4000:], flush=True)
    assert result.returncode == 0 and "static capture ok" in result.stdout
