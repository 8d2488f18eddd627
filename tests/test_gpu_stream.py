"""The context's stream binding (include/nva.h nva_ctx_set_stream): the mirror's Context runs
the library on torch's current stream, so library kernels are ordered with the caller's torch
copies and reads.  Torch's default stream is the null stream (handle 0), which the library
must take as HIP's null stream rather than as its own stream."""
import sys

import numpy as np
import pytest
import torch

from nanollvm_amd import Context, RMSNorm
from nanollvm_amd import _native as N

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def current(ctx):
    return N.load().nva_ctx_stream(ctx.handle) or 0


def test_context_runs_on_torch_current_stream():
    say("stream: default stream binding")
    c = Context(0)
    try:
        assert current(c) == torch.cuda.current_stream(0).cuda_stream
    finally:
        c.close()
    say("stream: explicit stream binding")
    s = torch.cuda.Stream(device=0)
    c = Context(0, stream=s)
    try:
        assert current(c) == s.cuda_stream
        x = torch.randn(4096, 1024, device="cuda")
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            out = RMSNorm.weightless(1e-6).forward(x, c)
            got = out.cpu().numpy()
        xh = x.cpu().numpy().astype(np.float64)
        ref = xh / np.sqrt((xh * xh).mean(axis=1, keepdims=True) + 1e-6)
        assert np.abs(got - ref).max() < 1e-5
    finally:
        c.close()


def test_outputs_read_right_after_the_call_are_complete():
    """Many back-to-back norms, each read back at once on torch's default stream."""
    say("stream: default-stream read-back")
    c = Context(0)
    try:
        norm = RMSNorm.weightless(0.0)
        for i in range(20):
            x = torch.full((2048, 512), float(i + 1), device="cuda")
            got = norm.forward(x, c).cpu().numpy()
            # sum of squares 512 v^2 and mean v^2 are exact; inv = (float)(1 / sqrt(v^2)).
            want = np.float32(i + 1) * np.float32(1.0 / np.sqrt(np.float64((i + 1) ** 2)))
            assert np.all(got == want), i
    finally:
        c.close()
