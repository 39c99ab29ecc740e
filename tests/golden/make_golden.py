"""Write golden vectors by running the reference implementation itself.

Runs N01N9/hdcmamba's own code (hdcmamba/model.py: its constructor, the
FusedNormConv1dFunction path, the full HdcMamba9v3Block forward and a two-block
HdcMamba9v3Model forward with its Triton kernels executed by Triton's CPU interpreter,
TRITON_INTERPRET=1) on small seeded
inputs, and saves inputs, weights, captured intermediates and outputs as plain tensor
files (torch.save of dicts of tensors; load with weights_only=True).  Nothing of the
reference's code is copied into the fixtures: they hold data only.

Usage (where the reference checkout is present; running the tests does not need it):
    python tests/golden/make_golden.py /path/to/reference

The reference's CPU launch-config branch returns keys its forward never reads
(model.py:13-14 vs 349), so each block instance gets the launch table the reference
uses on compute capability >= 8 (model.py:17) before its forward.

The interpreter keeps bf16 values as their uint16 bit patterns and its tl.dot multiplies
those integers (values of order 1e9 for inputs of order 1).  This script widens bf16 dot
operands to fp32 (exact) before the product, with fp32 accumulation, as a GPU's bf16 dot
computes it; every cast the reference's kernels make stays theirs, so the bf16 block
vectors record where the reference rounds.  The interpreter's fp32 -> bf16 cast truncates
(a GPU rounds to nearest even); the tests compare with the oracle in that rounding mode.
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

os.environ["TRITON_INTERPRET"] = "1"

HERE = Path(__file__).resolve().parent


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import torch
    import triton

    from hdcmamba.model import (FusedNormConv1dFunction, HdcMamba9v3Block)

    import numpy as np
    import triton.language as tl
    from triton.runtime import interpreter as tri_interp

    plain_dot = tri_interp.InterpreterBuilder.create_dot

    def dot_widening_bf16(self, a, b, d, input_precision, max_num_imprecise_acc):
        if a.dtype != tl.bfloat16 and b.dtype != tl.bfloat16:
            return plain_dot(self, a, b, d, input_precision, max_num_imprecise_acc)

        def widen(h):
            if h.dtype == tl.bfloat16:
                return (h.data.astype(np.uint32) << 16).view(np.float32)
            return h.data.astype(np.float32)

        acc = np.matmul(widen(a), widen(b), dtype=np.float32)
        return tri_interp.TensorHandle(acc + d.data, d.dtype.scalar)

    tri_interp.InterpreterBuilder.create_dot = dot_widening_bf16

    def cfg_for(blk):
        nb = lambda v, lo: max(lo, triton.next_power_of_2(v))  # noqa: E731
        return {"ssm_block_d": nb(blk.d_state, 64), "ssm_warps": 8, "slot_block_c": 128,
                "slot_block_d": nb(blk.head_dim, 64), "slot_warps": 8,
                "out_block_d_state": nb(blk.d_state, 64), "out_block_d_head": nb(blk.head_dim, 64),
                "out_warps": 8}

    out = {}

    # 1. Seeded construction: the parameters the constructor draws (RNG order).
    for seed, (dm, ds, H, C) in [(0, (64, 16, 2, 64)), (1, (96, 16, 3, 32)), (2, (64, 32, 4, 256))]:
        torch.manual_seed(seed)
        blk = HdcMamba9v3Block(d_model=dm, d_state=ds, num_heads=H, chunk_size=C)
        out[f"ctor_{seed}"] = {"args": torch.tensor([dm, ds, H, C, seed]),
                               **{k: v.detach().clone() for k, v in blk.state_dict().items()}}

    # 2. FusedNormConv1dFunction (LayerNorm + causal conv) forward, fp32 and bf16.
    for dt_name, dt in (("f32", torch.float32), ("bf16", torch.bfloat16)):
        g = torch.Generator().manual_seed(11)
        D = 64
        x = (2 * torch.randn(2, 37, D, generator=g) + 0.3).to(dt)
        w = (1 + 0.2 * torch.randn(D, generator=g)).to(dt)
        b = (0.2 * torch.randn(D, generator=g)).to(dt)
        cw = (0.3 * torch.randn(D, 4, generator=g)).to(dt)
        cb = (0.1 * torch.randn(D, generator=g)).to(dt)
        y = FusedNormConv1dFunction.apply(x, w, b, cw, cb, 1e-5)
        out[f"norm_conv_{dt_name}"] = {"x": x, "ln_w": w, "ln_b": b, "conv_w": cw, "conv_b": cb, "out": y}

    # 3. Full block forwards (eval) with captured intermediates.
    cases = {
        # name: (d_model, d_state, heads, chunk, B, L, dtype)
        "block_h64_c64": (64, 16, 1, 64, 1, 128, torch.float32),
        "block_h32_c64_b2": (64, 16, 2, 64, 2, 192, torch.float32),
        "block_h64_c128": (64, 16, 1, 128, 1, 256, torch.float32),
        "block_h96_c32": (96, 16, 1, 32, 1, 128, torch.float32),
        "block_h64_c64_pad": (64, 16, 1, 64, 1, 100, torch.float32),
        # bf16 (the dots widened as above): the slot recurrence's rounding points
        "block_h64_c64_bf16": (64, 16, 1, 64, 1, 192, torch.bfloat16),
        "block_h32_c64_b2_bf16": (64, 16, 2, 64, 2, 128, torch.bfloat16),
    }
    for i, (name, (dm, ds, H, C, B, L, dt)) in enumerate(cases.items()):
        torch.manual_seed(100 + i)
        blk = HdcMamba9v3Block(d_model=dm, d_state=ds, num_heads=H, chunk_size=C)
        g = torch.Generator().manual_seed(200 + i)
        with torch.no_grad():  # non-trivial norm / group-norm affine and per-head decays
            blk.norm.weight.copy_(1 + 0.1 * torch.randn(dm, generator=g))
            blk.norm.bias.copy_(0.1 * torch.randn(dm, generator=g))
            blk.group_norm.weight.copy_(1 + 0.1 * torch.randn(dm, generator=g))
            blk.group_norm.bias.copy_(0.1 * torch.randn(dm, generator=g))
            blk.decay_log.copy_(torch.log(1.0 / (0.9 + 0.09 * torch.rand(H, generator=g)) - 1.0))
            blk.gamma_buf.copy_(torch.exp(-torch.nn.functional.softplus(blk.decay_log)))
        blk = blk.eval().to(dt)
        blk.triton_cfg = cfg_for(blk)
        cap = {}
        h1 = blk.in_proj.register_forward_hook(lambda m, a, o: cap.__setitem__("projs", o.detach().clone()))
        h2 = blk.out_proj.register_forward_pre_hook(lambda m, a: cap.__setitem__("combined_ln", a[0].detach().clone()))
        x = torch.randn(B, L, dm, generator=g).to(dt)
        with torch.no_grad():
            y, _ = blk(x)
        h1.remove(); h2.remove()
        out[name] = {"args": torch.tensor([dm, ds, H, C, B, L]), "x": x, "y": y, **cap,
                     **{"p." + k: v.detach().clone() for k, v in blk.state_dict().items()}}
        print(name, "done", flush=True)

    # 4. The three SSM kernels launched as _inner_forward launches them (model.py:345-363),
    #    fp32 and bf16: intra-chunk scan, chunk carry, inter-chunk correction.
    import hdcmamba.model as R
    for dt_name, dt in (("f32", torch.float32), ("bf16", torch.bfloat16)):
        g = torch.Generator().manual_seed(21)
        B, L, ds, C = 2, 192, 16, 64
        N = L // C
        projs = torch.randn(B, L, 3 * ds + 8, generator=g)
        projs[..., :ds] = torch.log(torch.expm1(0.001 + 0.099 * torch.rand(B, L, ds, generator=g)))
        projs = projs.to(dt)
        A_log = torch.log(torch.linspace(0.99, 0.9999, ds)).to(dt)
        y = torch.empty(B, N, C, ds, dtype=dt)
        last = torch.empty(B, N, ds, dtype=dt)
        cd, G = torch.empty_like(last), torch.empty_like(last)
        R._ssm_intra_v2[(B, N)](projs, y, last, cd, A_log, *projs.stride(), *y.stride(), *last.stride(),
                                D_STATE=ds, CHUNK_SIZE=C, BLOCK_SIZE_D=64)
        R._ssm_scan_v2[(B,)](last, G, cd, *last.stride(), N=N, D_STATE=ds)
        R._ssm_inter_v2[(B, N)](projs, y, G, A_log, *projs.stride(), *y.stride(), *G.stride(),
                                D_STATE=ds, CHUNK_SIZE=C, BLOCK_SIZE_D=64)
        out[f"ssm_{dt_name}"] = {"args": torch.tensor([B, L, ds, C]), "projs": projs, "A_log": A_log,
                                 "y": y.view(B, L, ds).clone()}

    # 5. The model forward (model.py:396-404): two blocks chained through the residual stream,
    #    then norm_final, fp32.  The reference's model builds its blocks with chunk 256, which
    #    its slot kernels cannot run (model.py:17,245-246: rows past the 128-row tile are never
    #    written), so the blocks are switched to chunk 64 before the forward.
    from hdcmamba.model import HdcMamba9v3Model
    torch.manual_seed(300)
    m = HdcMamba9v3Model(d_model=64, n_layers=2, d_state=16, num_slots=32, num_heads=2)
    g = torch.Generator().manual_seed(301)
    with torch.no_grad():
        for blk in m.layers:
            blk.chunk_size = 64
            blk.group_norm.weight.copy_(1 + 0.1 * torch.randn(64, generator=g))
            blk.decay_log.copy_(torch.log(1.0 / (0.9 + 0.09 * torch.rand(2, generator=g)) - 1.0))
            blk.gamma_buf.copy_(torch.exp(-torch.nn.functional.softplus(blk.decay_log)))
        m.norm_final.weight.copy_(1 + 0.1 * torch.randn(64, generator=g))
        m.norm_final.bias.copy_(0.1 * torch.randn(64, generator=g))
    m = m.eval()
    for blk in m.layers:
        blk.triton_cfg = cfg_for(blk)
    x = torch.randn(1, 100, 64, generator=g)
    with torch.no_grad():
        y = m(x)
    out["model_2l"] = {"args": torch.tensor([64, 16, 2, 64, 1, 100, 2]), "x": x, "y": y,
                       **{"p." + k: v.detach().clone() for k, v in m.state_dict().items()}}
    print("model_2l done", flush=True)

    path = HERE / "reference_vectors.pt"
    torch.save(out, path)
    print("wrote", path, path.stat().st_size, "bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
