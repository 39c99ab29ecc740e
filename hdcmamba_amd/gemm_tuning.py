"""hipBLASLt solution selection for the block's GEMMs (in_proj, out_proj, tied LM head).

The projections stay library GEMMs; what this module changes is which hipBLASLt solution
runs them.  PyTorch's TunableOp benchmarks every hipBLASLt/rocBLAS solution for a GEMM
signature (transposes, M, N, K, leading dimensions, bias) and records the fastest in a CSV
file whose header pins the PyTorch, HIP, hipBLASLt and rocBLAS versions and the GPU
architecture.  ``use_tuned_gemms()`` loads the file shipped beside this module with tuning
switched off: a recorded signature runs its recorded solution, any other GEMM runs the
library's default heuristic, and a file written under other versions is ignored by
TunableOp's validators.

    python -m hdcmamba_amd.gemm_tuning --out hdcmamba_amd/tuned/gemm_gfx950.csv

re-tunes the signatures of the workloads listed in WORKLOADS (one block per model size is
enough: every block has the same shapes) on the current GPU and writes the file.
"""
from __future__ import annotations

import argparse
import os
from pathlib import Path

import torch

TUNED_FILE = Path(__file__).resolve().parent / "tuned" / "gemm_gfx950.csv"

# (d_model, d_state, num_heads, vocab, chunk, forward (B, L) list, prefill/decode (B, L) or None)
WORKLOADS = {
    "d768": (768, 64, 12, 50304, 64, [(8, 4096), (2, 512)], None),
    "d1024": (1024, 128, 16, 50304, 64, [(1, 32768)], None),
    "d2048": (2048, 128, 32, 50304, 64, [], (16, 8192)),
}


def use_tuned_gemms(path: os.PathLike | str | None = None) -> int:
    """Enable TunableOp with tuning off and load the recorded solutions.  Returns the
    number of GEMM signatures loaded (0 when the file is missing or its versions do not
    match this process)."""
    path = Path(path) if path is not None else TUNED_FILE
    if not path.exists():
        return 0
    tun = torch.cuda.tunable
    tun.enable(True)
    tun.tuning_enable(False)
    if not tun.read_file(str(path)):
        return 0
    return len(tun.get_results())


def _tune(out: Path, names) -> None:
    from .lm import HdcMambaLM

    tun = torch.cuda.tunable
    tun.enable(True)
    tun.tuning_enable(True)
    tun.set_filename(str(out), insert_device_ordinal=False)
    # candidates are timed over rotating copies of the operands (512 MB), so a solution is
    # judged with cold caches as it runs inside a forward, not on operands left in the
    # 256 MB last-level cache by its previous repetition
    tun.set_rotating_buffer_size(512)
    dev = torch.device("cuda:0")
    for name in names:
        dm, ds, H, V, C, fwd, pre = WORKLOADS[name]
        torch.manual_seed(0)
        lm = HdcMambaLM(dm, 1, ds, H, vocab_size=V, chunk_size=C).eval().to(torch.bfloat16).to(dev)
        with torch.no_grad():
            for B, L in fwd:
                ids = torch.randint(0, V, (B, L), device=dev)
                lm(ids)
                print(f"tuned {name} forward B={B} L={L}", flush=True)
            if pre is not None:
                B, L = pre
                ids = torch.randint(0, V, (B, L + 2), device=dev)
                _, states = lm.prefill(ids[:, :L])
                lm.step(ids[:, L].contiguous(), states)
                print(f"tuned {name} prefill B={B} L={L} and decode", flush=True)
        del lm
        torch.cuda.empty_cache()
    # TunableOp writes the file when the process exits


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--out", default=str(TUNED_FILE))
    ap.add_argument("--workloads", nargs="*", default=list(WORKLOADS))
    args = ap.parse_args()
    out = Path(args.out)
    out.parent.mkdir(parents=True, exist_ok=True)
    _tune(out, args.workloads)
    print(f"wrote {out}")


if __name__ == "__main__":
    main()
