"""Pre-selected hipBLASLt / rocBLAS solutions for the GEMMs around the scan.

The layer's projections and the LM's MLP and head are plain library GEMMs (torch
``matmul`` -> hipBLASLt). hipBLASLt's default heuristic does not always pick its fastest
solution at these shapes. PyTorch's TunableOp times every solution of hipBLASLt and
rocBLAS for a shape and records the fastest in a CSV; with that file loaded (and tuning
off) each GEMM of a recorded shape runs the recorded solution, and any other shape runs
the default. The file is keyed by the library versions it was made with (its
``Validator`` rows): on other versions torch ignores it.

    python mamba3-siso-tpu_amd/gemm_tuning.py tune [PATH]   # on the GPU: regenerate
    gemm_tuning.enable()                                      # use the committed file

`tune` runs, once each, the workloads whose GEMM shapes the benchmark measures: the
configs[1]/[2] layer forward and backward (B=8, L=8192, d_model=1024), the configs[3]
decode step (B=256), the configs[4] LM training step (B=16, L=2048, d_model=768) and the
LM's decode step at batch 1 and 256. Results are numerically the GEMMs' own:
only the choice of library kernel changes.
"""

from __future__ import annotations

import os
import sys

import torch

TUNED_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tuned_gemms.csv")


def enable(path: str = TUNED_FILE) -> bool:
    """Use the solutions recorded in ``path`` for the GEMMs of recorded shapes (tuning
    stays off, so nothing is timed at run time). Returns False if the file is missing or
    was not read."""
    if not os.path.exists(path):
        return False
    torch.cuda.tunable.enable(True)
    torch.cuda.tunable.tuning_enable(False)
    return bool(torch.cuda.tunable.read_file(path))


def disable() -> None:
    torch.cuda.tunable.enable(False)


def _workloads(m3, dev):
    """One pass of each benchmarked workload (its GEMMs are what gets tuned)."""
    cfg = m3.SISOConfig(d_model=1024, d_state=128, headdim=64, expand=2, chunk=128)
    p32 = m3.init_params(cfg, 0, device=dev)
    p16 = p32._replace(in_proj=p32.in_proj.to(torch.bfloat16),
                       out_proj=p32.out_proj.to(torch.bfloat16))
    u = torch.randn(8, 8192, 1024, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        m3.mamba3_siso_layer(p16, u, cfg)
        # the layer's decode step at B=256 (its two projections are small GEMMs)
        state = m3.zero_state(256, cfg.nheads, cfg.headdim, cfg.d_state, cfg.n_angles)
        state = m3.SISOState(*(t.to(dev) for t in state))
        m3.mamba3_siso_decode_step(p16, torch.randn(256, 1024, device=dev).to(torch.bfloat16),
                                   cfg, state)
    pg = m3.SISOParams(*(t.detach().clone().requires_grad_(True) for t in p32))
    ug = u.detach().clone().requires_grad_(True)
    y, _ = m3.mamba3_siso_layer(pg, ug, cfg)
    y.backward(torch.randn_like(y))
    del pg, ug, y
    T = m3.train
    scfg = m3.SISOConfig(d_model=768, d_state=128, headdim=64, expand=2, chunk=128)
    lcfg = m3.model.LMConfig(vocab_size=256, n_layers=8, siso=scfg, tie_head=True,
                             d_intermediate=1536)
    params = T.train_params(m3.model.init_lm(lcfg, 0, device=dev))
    opt = T.make_optimizer(params, lr=1e-3, warmup=100, steps=2000)
    step = T.make_step(lcfg, opt)
    xs = torch.randint(0, 256, (16, 2048), device=dev)
    step(params, opt, xs, xs)
    # the LM's decode step at batch 1 and 256 (its products are matrix-vector shapes)
    dparams = m3.model.decode_params(params, lcfg)
    with torch.no_grad():
        for bsz in (1, 256):
            states = m3.model.zero_states(lcfg, bsz, device=dev)
            m3.model.lm_decode_step(dparams, torch.zeros(bsz, dtype=torch.int64, device=dev),
                                    states, lcfg)
    torch.cuda.synchronize()


def tune(path: str = TUNED_FILE, max_ms_per_gemm: int = 400) -> None:
    """Time every library solution of each GEMM shape the workloads run and record the
    fastest in ``path`` (written when the process exits). Needs the GPU."""
    here = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    if here not in sys.path:
        sys.path.insert(0, here)
    import __graft_entry__

    m3 = __graft_entry__.load_package()
    torch.cuda.tunable.enable(True)
    torch.cuda.tunable.tuning_enable(True)
    torch.cuda.tunable.set_filename(path)
    torch.cuda.tunable.set_max_tuning_duration(max_ms_per_gemm)
    _workloads(m3, torch.device("cuda:0"))
    print(f"tuned {len(torch.cuda.tunable.get_results())} GEMM shapes -> {path}", flush=True)


if __name__ == "__main__":
    if len(sys.argv) < 2 or sys.argv[1] != "tune":
        raise SystemExit("usage: gemm_tuning.py tune [PATH]")
    tune(sys.argv[2] if len(sys.argv) > 2 else TUNED_FILE)
