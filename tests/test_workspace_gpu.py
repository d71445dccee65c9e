"""Library-owned GEMM workspaces are per (device, stream): two streams in flight at once on one GPU each get their own
split-K partials and pre-pass buffers, so every result equals the same call made serially (the reference keeps these
buffers thread_local, src/kernels/gemm.cu:3258-3368)."""
import pytest
import torch

from qengine_amd import call, ops, synth
from test_gemm_gpu import SPLIT_SHAPE, setup

pytestmark = pytest.mark.gpu

KIND = {"split": 0, "i8": 1, "h16": 2}


def _run(path, w, x):
    if path == "i8":
        return ops.gemm_w4_i8(w, x, G=64)
    if path == "h16":
        return ops.gemm_w4h(w, x)
    return ops.gemm_w4_choice(w, x, cfg=0, ks=2)[0]


@pytest.mark.parametrize("path", ["i8", "h16", "split"])
def test_two_streams_keep_their_own_workspace(dev, path):
    n, k, t = SPLIT_SHAPE if path == "split" else (4096, 2048, 700)
    w, _, _ = setup(n, k, 1, seed=n + t)
    xs = [synth.to_dev(synth.x_host(t, k, seed=s)) for s in (1, 2)]
    want = [_run(path, w, x) for x in xs]  # serial, default stream
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:  # size each stream's buffers with an eager call before the overlapped ones
        with torch.cuda.stream(s):
            _run(path, w, xs[0])
    torch.cuda.synchronize()
    got = [[], []]
    for _ in range(8):  # the two streams' calls interleaved, nothing waits in between
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                got[i].append(_run(path, w, xs[i]))
    torch.cuda.synchronize()
    iv = torch.int16 if want[0].dtype == torch.bfloat16 else torch.int32
    for i in range(2):
        for r, y in enumerate(got[i]):
            assert torch.equal(y.view(iv), want[i].view(iv)), (path, i, r)
    assert call("qe_workspace_count", KIND[path]) >= 3  # the default stream's and one per stream
