"""hdcm_ssm_fwd_noalloc (the scan on the library's fixed per-GPU scratch) through the C ABI
against hdcm_ssm_fwd (the same kernels on an allocated workspace): calls in a row on the scratch
as earlier calls left it (a smaller input second, then inputs whose look-back reads tile totals
over words of earlier calls), each bit-identical to the workspace entry point's result on a
freshly zeroed workspace; and, in a fresh process, a first call recorded in a HIP graph and
replayed."""
import os
import subprocess
import sys

import pytest
import torch

from cfgs import ssm_inputs
from hdcmamba_amd import _ops

pytestmark = pytest.mark.gpu

ETOOBIG = -6


def _call(fn_name, projs, A_log, ds, y, hf, ws=None):
    lib = _ops.lib()
    B, L, P = projs.shape
    stream = torch.cuda.current_stream(projs.device).cuda_stream
    args = [projs.data_ptr(), P, A_log.data_ptr(), None, y.data_ptr(), y.stride(1), hf.data_ptr(), None, 0]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    args += [B, L, ds, _ops._dtype(projs), stream]
    return getattr(lib, fn_name)(*args)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry_point(dev, dtype):
    lib = _ops.lib()
    # the second call is smaller; the third repeats the first shape with other data (its tile
    # totals land on words the first call tagged), the fourth reads three tiles' totals
    for k, (B, L, ds) in enumerate(((2, 1000, 128), (1, 300, 64), (2, 1000, 128), (1, 1500, 64))):
        print("ssm noalloc", dtype, B, L, ds, flush=True)
        projs, A_log = ssm_inputs(B, L, ds, dtype, seed=L + 7 * k)
        projs, A_log = projs.to(dev), A_log.to(dev)
        y_ref = torch.zeros(B, L, ds + 8, device=dev, dtype=dtype)
        hf_ref = torch.zeros(B, ds, device=dev)
        ws = torch.zeros(lib.hdcm_ssm_workspace_bytes(B, L, ds), dtype=torch.uint8, device=dev)  # zero before first use
        assert _call("hdcm_ssm_fwd", projs, A_log, ds, y_ref[..., :ds], hf_ref, ws) == 0
        y = torch.zeros_like(y_ref)
        hf = torch.zeros_like(hf_ref)
        assert _call("hdcm_ssm_fwd_noalloc", projs, A_log, ds, y[..., :ds], hf) == 0
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), (y.float() - y_ref.float()).abs().max().item()
        assert torch.equal(hf, hf_ref)
        assert y[..., ds:].abs().max().item() == 0.0


def test_noalloc_rejects_inputs_beyond_its_scratch(dev):
    lib = _ops.lib()
    B, L, ds = 256, 32768, 128  # tile totals: 256 x 128 channels x 64 tiles x 16 B = 32 MiB of scratch
    assert lib.hdcm_ssm_workspace_bytes(B, L, ds) > (8 << 20)
    projs = torch.empty(16, dtype=torch.bfloat16, device=dev)  # never read: rejected first
    st = lib.hdcm_ssm_fwd_noalloc(projs.data_ptr(), 3 * ds, projs.data_ptr(), None, projs.data_ptr(), ds, None,
                                  None, 0, B, L, ds, _ops.HDCM_BF16, torch.cuda.current_stream(dev).cuda_stream)
    assert st == ETOOBIG
    assert b"scratch" in lib.hdcm_strerror(st)


def test_noalloc_first_call_under_graph_capture(dev):
    """The first call of a process, made while torch.cuda.graph records it, looks up the scratch
    address and is recorded; replays with new inputs match hdcm_ssm_fwd bit for bit."""
    script = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_capture_check.py")
    print("ssm noalloc under capture (child process)", flush=True)
    r = subprocess.run([sys.executable, "-u", script], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stdout + r.stderr[-2000:]
    assert "capture ok" in r.stdout
