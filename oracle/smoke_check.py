"""`__graft_entry__.smoke()`'s check: one small layer forward + backward and one decode
step on cuda:0 through the HIP kernels, compared with this oracle. Test
infrastructure only (the oracle is the checker, never the thing run)."""

from __future__ import annotations

import torch

from . import siso_oracle as O


def run(m3) -> None:
    if not torch.cuda.is_available():
        raise RuntimeError("smoke() needs a ROCm device")
    dev = torch.device("cuda:0")
    cfg = m3.SISOConfig(d_model=64, d_state=16, headdim=16, expand=1, chunk=64, policy_name="f32")
    p_cpu = m3.init_params(cfg, 0)
    u = torch.randn(1, 256, 64, generator=torch.Generator().manual_seed(0))
    gy = torch.randn(1, 256, 64, generator=torch.Generator().manual_seed(1))

    params = m3.SISOParams(*(t.to(dev).requires_grad_(True) for t in p_cpu))
    ud = u.to(dev).requires_grad_(True)
    y, st = m3.mamba3_siso_layer(params, ud, cfg)
    (y * gy.to(dev)).sum().backward()

    pd = {f: getattr(p_cpu, f).double().requires_grad_(True) for f in p_cpu._fields}
    uo = u.double().requires_grad_(True)
    yr, sr = O.layer_forward(pd, uo, d_state=16, headdim=16, expand=1, chunk=64)
    (yr * gy.double()).sum().backward()

    checks = {
        "y": O.rel_error(y.detach().cpu(), yr.detach()),
        "final ssm": O.rel_error(st.ssm.detach().cpu(), sr.ssm.detach()),
        "du": O.rel_error(ud.grad.cpu(), uo.grad),
        "d in_proj": O.rel_error(params.in_proj.grad.cpu(), pd["in_proj"].grad),
        "d dt_bias": O.rel_error(params.dt_bias.grad.cpu(), pd["dt_bias"].grad),
    }
    # one decode step from the prefill's carry
    tok = torch.randn(1, 64, generator=torch.Generator().manual_seed(2))
    carry = O.SISOState(*(t.detach().cpu().double() for t in st))
    yd, _ = m3.mamba3_siso_decode_step(
        m3.SISOParams(*(t.detach() for t in params)), tok.to(dev), cfg,
        m3.SISOState(*(t.detach().clone() for t in st)))
    ydr, _ = O.layer_decode_step({f: getattr(p_cpu, f).double() for f in p_cpu._fields},
                                 tok.double(), carry, d_state=16, headdim=16, expand=1)
    checks["decode y"] = O.rel_error(yd.cpu(), ydr)
    tol = {"y": 2e-5, "final ssm": 2e-5, "du": 2e-4, "d in_proj": 2e-4, "d dt_bias": 2e-4,
           "decode y": 1e-4}
    bad = {k: v for k, v in checks.items() if not v <= tol[k]}
    print("smoke:", ", ".join(f"{k} {v:.1e}" for k, v in checks.items()))
    if bad:
        raise AssertionError(f"smoke parity failed: {bad}")
