"""Shared helpers for the GPU parity tests: identical seeded inputs for the CPU oracle
(float64) and the device (policy dtype), and the tolerance checks.

Tolerances (stated once, used by every GPU test):
  * f32 policy vs the float64 oracle: p95 relative error over |ref| >= 1e-2
    (``tests.py:60-88``) <= 2e-5 for forward/decode outputs and <= 2e-4 for gradients
    (the reference's own bars, ``tests.py:533, 612``), AND max |got - ref| / max |ref|
    <= 1e-4 on outputs and <= 1e-3 on gradients (`assert_f32`). The p95 figure alone
    ignores the worst 5% of entries and every entry below 1e-2, so a wrong row per chunk
    or an unwritten tile could pass it; the max-normalised bound catches those.
  * bf16 policy against the oracle's bf16 rounding model (the same rounding points as the
    reference kernel): p95 <= 2e-3 for f32 outputs (the state) and <= 5e-3 for outputs
    stored in bf16 (y, and ybar, which the bf16 policy stores in bf16; one bf16 rounding
    is up to 2^-8 relative); elementwise, a bf16
    output is within one bf16 ulp of |ref| plus 4e-3 max|ref| (the operand roundings of
    the products, which the model reproduces only up to accumulation order).
  * bf16 policy against the float64 maths:
      - max |got - ref| / max |ref| <= 1e-2 on outputs (y);
      - max |got - ref| <= 2e-2 on the float32 final state (the north_star bound);
      - max |got - ref| / max |ref| <= 2e-2 on every gradient (north_star: 5e-2);
      - p95 <= 5e-2 on the kernel's y, the reference's bf16 bar (``tests.py:533``).
    At the layer level the bf16 projections round the weights and every stored
    activation (``layer.py:233, 256``); the layer's y is held to the rounding model of the
    whole bf16 layer (`siso_oracle.layer_forward(act_dtype=bf16)`), p95 <= 1e-2.
"""

import torch

from oracle import siso_oracle as O

F64 = torch.float64
F32 = torch.float32
BF16 = torch.bfloat16

FWD_F32_P95 = 2e-5
GRAD_F32_P95 = 2e-4
F32_OUT_MAXREL = 1e-4
F32_GRAD_MAXREL = 1e-3
BF16_MODEL_P95 = 2e-3
BF16_OUT_MODEL_P95 = 5e-3
BF16_LAYER_MODEL_P95 = 1e-2
BF16_Y_MAXREL = 1e-2
BF16_MAXREL = 2e-2
BF16_GRAD_MAXREL = 2e-2
BF16_P95 = 5e-2
STATE_MAXABS = 2e-2
BF16_MODEL_ABS_REL = 4e-3


def mt_of(policy):
    return BF16 if policy == "bf16" else F32


def boundary_inputs(b, h, seqlen, n, p, nr, policy, seed=0, seeds=False):
    """Kernel-boundary inputs. Tensors the kernel reads in the policy dtype are rounded
    to it first, so oracle and kernel see identical values. Returns (cpu_f64, device)."""
    x = O.make_inputs(b, h, seqlen, n, p, nr, seed=seed)
    pre, _ = O.preprocess(x["dt_raw"], x["a_raw"], x["trap_raw"], x["angles"], x["dt_bias"])
    mt = mt_of(policy)
    cpu = dict(
        q=x["q"].to(mt).double(), k=x["k"].to(mt).double(), v=x["v"].to(mt).double(),
        z=x["z"].to(mt).double(), adt=pre.adt.float().double(), gamma=pre.gamma.float().double(),
        scale=pre.scale.float().double(), phi=pre.phi.float().double(),
        q_bias=x["q_bias"].float().double(), k_bias=x["k_bias"].float().double(),
        d_skip=x["d_skip"].float().double(), dy=x["dy"].to(mt).double(),
        dt=pre.dt.float().double(), lam=pre.lam.float().double(),
        angles=x["angles"].float().double())
    if seeds:
        g = torch.Generator().manual_seed(seed + 1000)
        cpu.update(
            seed_ssm=torch.randn(b, h, p, n, generator=g, dtype=F64).float().double(),
            seed_k=torch.randn(b, h, n, generator=g, dtype=F64).float().double(),
            seed_v=torch.randn(b, h, p, generator=g, dtype=F64).float().double(),
            seed_coef=torch.rand(b, h, generator=g, dtype=F64).float().double())
    dev = {}
    for k_, v_ in cpu.items():
        dt_ = mt if k_ in ("q", "k", "v", "z", "dy") else F32
        dev[k_] = v_.to(dt_).cuda()
    return cpu, dev


def fwd_args(d):
    return [d["q"], d["k"], d["v"], d["adt"], d["gamma"], d["scale"], d["phi"], d["q_bias"],
            d["k_bias"], d.get("d_skip"), d.get("z"), d.get("seed_ssm"), d.get("seed_k"),
            d.get("seed_v"), d.get("seed_coef")]


def cpu(t):
    return t.detach().float().cpu().double()


def report(what, got, ref):
    """Print the error figures of one comparison (visible with ``pytest -s``)."""
    g, r = cpu(got), ref.detach().double()
    print(f"[parity] {what}: p95 {O.rel_error(g, r):.3e}  max-norm {O.max_rel(g, r):.3e}  "
          f"max-abs {O.max_abs(g, r):.3e}  (max|ref| {float(r.abs().max()):.3e})", flush=True)


def assert_p95(got, ref, tol, what=""):
    e = O.rel_error(cpu(got), ref)
    assert e <= tol, f"{what}: p95 rel error {e:.3e} > {tol:.1e}"


def assert_maxrel(got, ref, tol, what=""):
    e = O.max_rel(cpu(got), ref)
    assert e <= tol, f"{what}: max-normalised error {e:.3e} > {tol:.1e}"


def assert_f32(got, ref, kind, what=""):
    """The f32 policy's two bars against the float64 oracle: the reference's p95 metric
    and a max-normalised bound over every entry (``kind`` "out": 2e-5 / 1e-4; "grad":
    2e-4 / 1e-3). A reference that is zero throughout needs |got| <= 1e-6."""
    p95, mx = (FWD_F32_P95, F32_OUT_MAXREL) if kind == "out" else (GRAD_F32_P95, F32_GRAD_MAXREL)
    g, r = cpu(got), ref.detach().double().cpu()
    assert bool(torch.isfinite(g).all()), f"{what}: non-finite entries"
    assert_p95(g, r, p95, what)
    top = float(r.abs().max()) if r.numel() else 0.0
    err = float((g - r).abs().max()) if r.numel() else 0.0
    if top < 1e-6:
        assert err <= 1e-6, f"{what}: reference ~0 but max |got| {err:.3e}"
    else:
        assert err <= mx * top, f"{what}: max-normalised error {err / top:.3e} > {mx:.1e}"


def assert_maxabs(got, ref, tol, what=""):
    e = O.max_abs(cpu(got), ref)
    assert e <= tol, f"{what}: max-abs error {e:.3e} > {tol:.1e}"


def bf16_ulp(x):
    """Spacing of bfloat16 numbers at |x| (8 significant bits); 2^-133 at zero."""
    e = torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -126)))
    return torch.pow(2.0, e - 7)


def assert_bf16_bound(got, ref, rel=BF16_MODEL_ABS_REL, what=""):
    """Elementwise |got - ref| <= ulp_bf16(|ref|) + rel * max|ref|: one rounding of the
    stored bf16 value plus the operand roundings of the products feeding it."""
    g, r = cpu(got), ref.detach().double()
    bound = bf16_ulp(r) + rel * float(r.abs().max())
    over = ((g - r).abs() / bound).max()
    assert float(over) <= 1.0, f"{what}: |err| reaches {float(over):.2f}x the bf16 bound"


def phi_strips_of(c, m3):
    """The compact phi (kernels.PhiStrips) of `boundary_inputs`' oracle preprocess, on the
    device: tanh(angles) pi, dt, and the angle entering each 16-token strip (the oracle's
    phi at token 16 s - 1; 0 for the first strip, since these inputs start from 0)."""
    b, h, l, nr = c["phi"].shape
    strips = torch.zeros(b, h, l // 16, nr, dtype=F64)
    strips[:, :, 1:] = c["phi"][:, :, 15:-1:16]
    return m3.kernels.PhiStrips((torch.tanh(c["angles"]) * torch.pi).float().cuda(),
                                c["dt"].float().cuda(), strips.float().cuda())
