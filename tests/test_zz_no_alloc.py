"""The allocation-free RMSNorm backward entry point
(kore_hip_rms_norm_backward_noalloc_f32, library-held scratch) against the
workspace entry point (kore_hip_rms_norm_backward_f32), through the C ABI:
bit-identical dx and dgamma on consecutive calls, the later ones smaller
than the first so stale scratch contents would show."""
import sys

import numpy as np
import pytest

from inputs import normal

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from kore_amd import _lib  # noqa: E402


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to("cuda:0")


def _run_pair(rows: int, cols: int, seed: int):
    print(f"no-alloc rms_norm_backward rows={rows} cols={cols} seed={seed}", flush=True)
    sys.stdout.flush()
    lib = _lib.load()
    dy, x = _dev(normal((rows, cols), seed)), _dev(normal((rows, cols), seed + 1))
    g = _dev(normal((cols,), seed + 2, 1.0, 0.02))
    stream = torch.cuda.current_stream().cuda_stream
    need = lib.kore_hip_rms_norm_backward_workspace_bytes(rows, cols)
    assert 0 < need <= lib.kore_hip_rms_norm_backward_noalloc_max_bytes()
    ws = torch.empty(need // 4 + 4, dtype=torch.float32, device="cuda:0")
    gx_ref, gg_ref = torch.empty_like(x), torch.empty_like(g)
    gx, gg = torch.full_like(x, float("nan")), torch.full_like(g, float("nan"))
    assert lib.kore_hip_rms_norm_backward_f32(dy.data_ptr(), x.data_ptr(), g.data_ptr(), gx_ref.data_ptr(),
                                              gg_ref.data_ptr(), ws.data_ptr(), ws.numel() * 4, rows, cols,
                                              1e-5, stream) == 0
    assert lib.kore_hip_rms_norm_backward_noalloc_f32(dy.data_ptr(), x.data_ptr(), g.data_ptr(), gx.data_ptr(),
                                                      gg.data_ptr(), rows, cols, 1e-5, stream) == 0
    torch.cuda.synchronize()
    assert gx.cpu().numpy().tobytes() == gx_ref.cpu().numpy().tobytes()
    assert gg.cpu().numpy().tobytes() == gg_ref.cpu().numpy().tobytes()


def test_no_alloc_first_call_under_graph_capture():
    """The first call on the device (when the library looks up its scratch
    array) made inside a HIP graph capture on a side stream: the capture
    succeeds, and every replay -- with eager work and synchronisation between
    replays -- gives dx and dgamma bit-identical to the workspace entry point.
    Collected first in this module, so the lookup has not run before it."""
    rows, cols = 300, 2560
    print(f"no-alloc rms_norm_backward under capture rows={rows} cols={cols}", flush=True)
    lib = _lib.load()
    dy, x = _dev(normal((rows, cols), 11)), _dev(normal((rows, cols), 12))
    g = _dev(normal((cols,), 13, 1.0, 0.02))
    need = lib.kore_hip_rms_norm_backward_workspace_bytes(rows, cols)
    ws = torch.empty(need // 4 + 4, dtype=torch.float32, device="cuda:0")
    gx_ref, gg_ref = torch.empty_like(x), torch.empty_like(g)
    assert lib.kore_hip_rms_norm_backward_f32(dy.data_ptr(), x.data_ptr(), g.data_ptr(), gx_ref.data_ptr(),
                                              gg_ref.data_ptr(), ws.data_ptr(), ws.numel() * 4, rows, cols,
                                              1e-5, torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    gx, gg = torch.full_like(x, float("nan")), torch.full_like(g, float("nan"))
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    rcs = []
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rcs.append(lib.kore_hip_rms_norm_backward_noalloc_f32(
                dy.data_ptr(), x.data_ptr(), g.data_ptr(), gx.data_ptr(), gg.data_ptr(), rows, cols, 1e-5,
                side.cuda_stream))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert rcs == [0]
    for rep in range(3):
        gx.fill_(float("nan"))
        gg.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gx, gx_ref), f"replay {rep}: dx"
        assert torch.equal(gg, gg_ref), f"replay {rep}: dgamma"


def test_no_alloc_matches_workspace_entry_point():
    # vector plan at full scratch use (512 partial rows x 2048), then smaller
    # vector plans, then the generic plan (cols % 4 != 0: per-row inv)
    _run_pair(16384, 2048, 1)
    _run_pair(100, 2048, 2)
    _run_pair(37, 256, 3)
    _run_pair(300, 1001, 4)
    _run_pair(5, 7, 5)


def test_no_alloc_rejects_work_beyond_scratch():
    lib = _lib.load()
    cap = lib.kore_hip_rms_norm_backward_noalloc_max_bytes()
    rows, cols = cap // 4 + 1, 3  # generic plan: one float per row
    assert lib.kore_hip_rms_norm_backward_workspace_bytes(rows, cols) > cap
    t = torch.zeros(4, device="cuda:0")
    p = t.data_ptr()
    assert lib.kore_hip_rms_norm_backward_noalloc_f32(p, p, p, p, p, rows, cols, 1e-5, None) == \
        _lib.KORE_HIP_ERR_SCRATCH
