"""Stream use of the library forward.  Captured in a HIP graph (torch.cuda.CUDAGraph, which
is hipGraph on ROCm) and replayed: every launch of the scan follows the
capturing stream and the forward allocates only through torch, so a serving
loop can replay the whole chunk loop of a layer as one graph.  Checked the
way graph use must be checked here: several replays, with eager work of the
program's own and synchronisations between them, each compared bitwise with
the eager result of the same inputs.  And two scans issued at once on two
streams, against the sequential results."""

import numpy as np
import pytest

import scan_cases as SC

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("precision,io", [("f16", "bf16"), ("f32", "f32")])
def test_forward_graph_replay(precision, io):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from atlas_amd import DeepMemoryState, memory_scan
    B, T, H, D, E, cs, w = 2, 256, 4, 64, 128, 64, 32
    inp = SC.make_inputs(B, T, H, D, E, seed=51, io=io, s_scale=0.05)
    tio = {"bf16": torch.bfloat16, "f32": torch.float32}[io]
    x = [torch.tensor(np.asarray(inp[n], np.float32), device="cuda").to(tio) for n in ("q", "k", "v")]
    gts = [torch.tensor(np.asarray(inp[n], np.float32), device="cuda") for n in ("alpha", "eta", "theta", "gamma")]
    st = DeepMemoryState(*(torch.tensor(s, dtype=torch.float32, device="cuda") for s in inp["state"]))

    def fwd():
        return memory_scan(*x, *gts, st, cs, w, 5, precision=precision)

    with torch.no_grad():
        y0, s0 = fwd()
        torch.cuda.synchronize()
        side = torch.cuda.Stream()   # default priority
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):   # warm-up off the default stream, as capture requires
            for _ in range(2):
                fwd()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            yg, sg = fwd()
        for r in range(3):
            junk = torch.randn(1024, 1024, device="cuda") @ torch.randn(1024, 1024, device="cuda")
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(yg, y0), f"replay {r}: y differs from the eager forward"
            for name, a, b in zip(("W1", "W2", "S1", "S2"), sg, s0):
                assert torch.equal(a, b), f"replay {r}: {name} differs from the eager forward"
            del junk


def test_concurrent_streams_forward():
    """Two layer scans issued at once on two torch streams (default
    priority) each allocate their own workspace through torch and share no
    device state: both results are bitwise the sequential ones."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from atlas_amd import DeepMemoryState, memory_scan
    B, T, H, D, E, cs, w = 4, 256, 8, 64, 128, 64, 32
    runs = []
    for seed in (61, 62):
        inp = SC.make_inputs(B, T, H, D, E, seed=seed, io="bf16", s_scale=0.05)
        x = [torch.tensor(np.asarray(inp[n], np.float32), device="cuda").to(torch.bfloat16) for n in ("q", "k", "v")]
        gts = [torch.tensor(np.asarray(inp[n], np.float32), device="cuda") for n in ("alpha", "eta", "theta", "gamma")]
        st = DeepMemoryState(*(torch.tensor(s, dtype=torch.float32, device="cuda") for s in inp["state"]))
        runs.append((x, gts, st))

    def fwd(r):
        x, gts, st = r
        return memory_scan(*x, *gts, st, cs, w, 5, precision="f16")

    with torch.no_grad():
        ref = [fwd(r) for r in runs]
        torch.cuda.synchronize()
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        for s in streams:
            s.wait_stream(torch.cuda.current_stream())
        out = []
        for s, r in zip(streams, runs):
            with torch.cuda.stream(s):
                out.append(fwd(r))
        for s in streams:
            torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
    for i, ((y, st), (y0, st0)) in enumerate(zip(out, ref)):
        assert torch.equal(y, y0), f"scan {i}: y differs when run concurrently"
        for name, a, b in zip(("W1", "W2", "S1", "S2"), st, st0):
            assert torch.equal(a, b), f"scan {i}: {name} differs when run concurrently"
