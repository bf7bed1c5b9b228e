"""GPU: seeai_xent_fwd_noalloc, the softmax cross-entropy forward that
allocates nothing (its row partials live in the library's file-scope device
workspace), against seeai_xent_fwd on the same inputs: loss and
probabilities bitwise equal, on two calls in a row (the second smaller, so
the workspace holds the first call's words when it starts), and a row count
past the workspace refused with a clear error."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _run(hip, ctx, torch, entry, logits, labels, masked):
    N, Cn = logits.shape
    dx = torch.from_numpy(logits).cuda()
    dl = torch.from_numpy(labels).cuda()
    loss = torch.full((1,), float("nan"), dtype=torch.float32, device="cuda")
    probs = torch.full((N, Cn), float("nan"), dtype=torch.float32, device="cuda")
    ctx.call(entry, dx.data_ptr(), dl.data_ptr(), loss.data_ptr(), probs.data_ptr(), N, Cn, masked)
    torch.cuda.synchronize()
    return loss.cpu().numpy(), probs.cpu().numpy()


@pytest.mark.parametrize("masked", [0, 1])
def test_xent_noalloc_matches_the_allocating_entry(hip, orc, torch_cuda, masked):
    torch = torch_cuda
    ctx = hip.Context(0)
    ctx.use_torch_stream()
    r = np.random.default_rng(17 + masked)
    for N, Cn in [(8192, 4000), (300, 1000)]:  # the second call is the smaller one
        print(f"no-alloc xent: N={N} C={Cn} masked={masked}", flush=True)
        logits = (r.standard_normal((N, Cn)) * 3).astype(np.float32)
        labels = r.integers(0, Cn, N).astype(np.int32)
        if masked:
            labels[::7] = -1
        want_loss, want_probs = _run(hip, ctx, torch, "seeai_xent_fwd", logits, labels, masked)
        got_loss, got_probs = _run(hip, ctx, torch, "seeai_xent_fwd_noalloc", logits, labels,
                                   masked)
        assert np.array_equal(got_loss.view(np.uint32), want_loss.view(np.uint32))
        assert np.array_equal(got_probs.view(np.uint32), want_probs.view(np.uint32))
        ref_loss, _ = orc.xent_fwd(logits, labels, masked=bool(masked))
        assert abs(float(got_loss[0]) - float(ref_loss)) <= 1e-5 * abs(float(ref_loss))
    ctx.close()


def test_xent_noalloc_refuses_rows_past_its_workspace(hip, torch_cuda):
    torch = torch_cuda
    ctx = hip.Context(0)
    n = hip.lib().seeai_xent_fwd_noalloc
    too_many = 131056 + 1
    dummy = torch.zeros(16, dtype=torch.float32, device="cuda")
    rc = n(ctx.h, C.c_void_p(dummy.data_ptr()), C.c_void_p(dummy.data_ptr()),
           C.c_void_p(dummy.data_ptr()), C.c_void_p(dummy.data_ptr()), too_many, 2, 0)
    assert rc == 2
    assert b"exceed" in hip.lib().seeai_last_error(ctx.h)
    ctx.close()
