"""Benchmark of the MI355X Mamba-3 SISO layer on BASELINE.json's workloads (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

The timed "step" is one layer forward at BASELINE configs[1] (B=8, L=8192, H=32, P=64,
N=128, d_model=1024, bf16, chunk 128; params from init_params(seed=0), u ~ N(0,1)
bf16): ``value`` is its tokens/s. The same run also measures, outside the K timed
steps, the forward+backward of configs[2] (dy ~ N(0,1) bf16, seed 2), the B=256 decode of
configs[3] (512 tokens), the scan kernel alone at the kernel boundary (the roofline
figure, timed with HIP events on the stream it is launched on), and the CPU oracle on a
bounded sample (``cpu_baseline``). Prints ONE JSON line.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
METRIC = "fwd & fwd+bwd tok/s @B8 H32 L8192 N128 P64 bf16; decode ms/token @B256"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--decode-tokens", type=int, default=512)
    ap.add_argument("--no-lm", action="store_true", help="skip the LM-stack legs")
    ap.add_argument("--default-gemms", action="store_true",
                    help="leave the library GEMMs on hipBLASLt's default heuristic instead of "
                         "the recorded solutions (gemm_tuning.enable)")
    ap.add_argument("--leg", choices=("all", "scan", "bwd", "decode", "copy", "lm", "wgrad"),
                    default="all",
                    help="run one leg alone (for rocprofv3 counter passes): 'scan' = the forward "
                         "scan kernel at the kernel boundary, 'bwd' = the backward scan kernel, "
                         "'decode' = the decode kernel, 'copy' = a plain 1 GiB device copy that "
                         "calibrates the FETCH_SIZE / WRITE_SIZE counters, 'lm' = the configs[4] "
                         "byte-LM training step and the LM decode stack, 'wgrad' = the "
                         "weight-gradient kernel at the configs[4] in_proj shape")
    return ap.parse_args()


def gpu_time_ms(fn, iters, torch):
    """Average GPU time of ``fn`` over ``iters`` back-to-back calls, measured with HIP
    events on the current stream (the stream every kernel here is launched on)."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def scan_inputs(m3, params16, cfg, u, torch):
    """Kernel-boundary operands of the configs[1] layer: the projections of ``u`` through
    split_in_proj and BCNorm, as the layer hands them to the scan. Three forms: raw mode
    (what the inference forward runs: the raw dt / a / trap slices of the projection and
    the rotary table and strip totals the BCNorm launch writes), the preprocess-fed scan
    with phi compact (``kernels.PhiStrips``), and the same phi materialised
    (``phi_full``, the training forward's form)."""
    from mamba3_siso_tpu_amd import kernels as K
    from mamba3_siso_tpu_amd import scan_prep as SP

    with torch.no_grad():
        proj = torch.nn.functional.pad(u @ params16.in_proj, (0, 128))   # the layer's padded row
        proj = proj[..., :cfg.d_in_proj]
        z, x, bb, cc, dt_raw, a_raw, trap_raw, angles = m3.split_in_proj(proj, cfg)
        bias = params16.dt_bias.float().contiguous()
        (kk, kq), _, angs = K.bcnorm_forward(
            [bb, cc], [params16.b_norm_weight, params16.c_norm_weight], cfg.norm_eps,
            theta=(angles, dt_raw, bias, cfg.chunk))
        adt, gamma, scale, _, _, strips, _ = SP.prep_forward_launch(
            dt_raw, a_raw, trap_raw, angles, bias, None, cfg.a_floor, compact=True)
        phi_full = SP.prep_forward_launch(dt_raw, a_raw, trap_raw, angles, bias, None,
                                          cfg.a_floor)[5]
        kv, kz = x.permute(0, 2, 1, 3), z.permute(0, 2, 1, 3)
    common = dict(q=kq, k=kk, v=kv, q_bias=params16.c_bias.float(),
                  k_bias=params16.b_bias.float(), d_skip=params16.d_skip.float(), z=kz)
    raw = dict(common, dt_raw=dt_raw, a_raw=a_raw, trap_raw=trap_raw, angles=angs,
               dt_bias=bias, a_floor=cfg.a_floor)
    return raw, dict(common, adt=adt, gamma=gamma, scale=scale, phi=strips), phi_full


def layer_roofline(B, L, DM, cfg, scan_bytes, scan_flops, measured_ms):
    """The layer forward's time floor: for each kernel, its algorithmic flops at the bf16
    MFMA peak or its algorithmic bytes at the HBM peak, whichever takes longer, summed
    over the kernels of the step; ``frac`` = floor / measured."""
    M, d_in, dpad = B * L, cfg.d_in_proj, (cfg.d_in_proj + 255) // 256 * 256
    H, N, Nr = cfg.nheads, cfg.d_state, cfg.n_angles

    def floor_ms(flops, nbytes):
        return max(flops / (BF16_PEAK_TFLOPS * 1e12), nbytes / (HBM_PEAK_GBS * 1e9)) * 1e3

    parts = {
        "in_proj": floor_ms(2 * M * DM * d_in, M * DM * 2 + DM * dpad * 2 + M * dpad * 2),
        # the B and C rows in and out; the angle and dt rows in, the rotary table and the
        # per-strip theta totals out (raw mode's share of the preprocess)
        "bcnorm": floor_ms(0, 4 * M * N * 2 + M * (H + Nr) * 2 + M * Nr * 4
                           + M * H * Nr * 4 // 16),
        "scan": floor_ms(scan_flops, scan_bytes),
        "out_proj": floor_ms(2 * M * cfg.d_inner * DM, M * cfg.d_inner * 2 + cfg.d_inner * DM * 2
                             + M * DM * 2),
    }
    floor = sum(parts.values())
    return {"floor_ms": round(floor, 4), "measured_ms": round(measured_ms, 4),
            "frac": round(floor / measured_ms, 4),
            "per_kernel_floor_ms": {k: round(v, 4) for k, v in parts.items()},
            "peaks": {"bf16_mfma_tflops": BF16_PEAK_TFLOPS, "hbm_gbs": HBM_PEAK_GBS}}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); every GPU box in "
              "this build has one GPU. The scan shards over (batch, head) with no "
              "communication: each GPU would run these kernels on its B/n share, and training "
              "would add one data-parallel all-reduce of the layer gradients.", file=sys.stderr)
        sys.exit(2)

    import torch
    import __graft_entry__

    m3 = __graft_entry__.load_package()
    from mamba3_siso_tpu_amd import gemm_tuning
    from mamba3_siso_tpu_amd import kernels as K

    # the library GEMMs around the scan run the hipBLASLt / rocBLAS solutions recorded for
    # these shapes (mamba3-siso-tpu_amd/tuned_gemms.csv); --default-gemms keeps hipBLASLt's
    # own heuristic
    tuned = False if args.default_gemms else gemm_tuning.enable()

    dev = torch.device("cuda:0")
    if args.leg == "copy":
        # 1 GiB read + 1 GiB written by one plain copy kernel: the FETCH_SIZE / WRITE_SIZE
        # calibration for the traffic figures.
        src = torch.empty(1 << 29, device=dev, dtype=torch.bfloat16).normal_()
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        ms = gpu_time_ms(lambda: dst.copy_(src), 10, torch)
        print(json.dumps({"leg": "copy", "bytes_read": 1 << 30, "bytes_written": 1 << 30,
                          "ms": round(ms, 4), "gbs": round(2 * (1 << 30) / (ms * 1e-3) / 1e9, 1)}))
        return

    if args.leg == "wgrad":
        # m3s_wgrad at the configs[4] in_proj weight gradient: u (B*L, 768) bf16 against
        # the projection gradient's 3432 used columns of a 3584-wide buffer
        gw = torch.Generator(device=dev).manual_seed(0)
        m, pw, qw, ldq = 16 * 2048, 768, 3432, 3584
        a = torch.randn(m, pw, generator=gw, device=dev).to(torch.bfloat16)
        b = torch.randn(m, ldq, generator=gw, device=dev).to(torch.bfloat16)[:, :qw]
        for _ in range(args.warmup + args.steps):
            K.wgrad(a, b)
        torch.cuda.synchronize()
        ms = min(gpu_time_ms(lambda: K.wgrad(a, b), max(args.steps, 10), torch) for _ in range(2))
        print(json.dumps({"leg": "wgrad", "shape": [m, pw, qw], "ms": round(ms, 4),
                          "tflops": round(2 * m * pw * qw / (ms * 1e-3) / 1e12, 1)}))
        return

    if args.leg == "lm":
        print(json.dumps({"leg": "lm", **lm_legs(m3, torch, dev)}))
        return

    B, L, H, P, N, DM = 8, 8192, 32, 64, 128, 1024
    cfg = m3.SISOConfig(d_model=DM, d_state=N, headdim=P, expand=2, chunk=128, policy_name="bf16")
    assert cfg.nheads == H
    Nr = cfg.n_angles
    params32 = m3.init_params(cfg, 0, device=dev)
    # weights resident in bf16 for the inference legs (the layer casts to u.dtype anyway)
    params16 = params32._replace(in_proj=params32.in_proj.to(torch.bfloat16),
                                 out_proj=params32.out_proj.to(torch.bfloat16))
    gen = torch.Generator(device=dev)
    u = torch.randn(B, L, DM, generator=gen.manual_seed(0), device=dev).to(torch.bfloat16)
    tokens = B * L
    line = {}

    # ---------------- the scan kernels alone, kernel boundary -------------------------
    # Algorithmic bytes of one forward launch as the layer's inference forward runs it
    # (raw mode): q, k once (head-shared), v, z, y bf16; the raw dt / a / trap slices bf16;
    # the tanh(angles) pi table (head-shared) and the theta strip totals f32; the final
    # ssm f32 (+ k, v, phi rows). The preprocess-fed scan reads adt / gamma / scale f32 and
    # phi compact (dt and one phi row per 16 tokens) or materialised (B, H, L, Nr) f32
    # (the training forward's form).
    phi_compact = B * L * Nr * 4 + B * H * L * 4 + B * H * (L // 16) * Nr * 4
    phi_read = B * H * L * Nr * 4
    scan_fixed = (2 * B * L * N * 2 + 3 * B * H * L * P * 2 + 3 * B * H * L * 4
                  + B * H * P * N * 4 + B * H * (N + P) * 4)
    scan_compact_bytes = scan_fixed + phi_compact
    scan_read_bytes = scan_fixed + phi_read
    scan_bytes = (2 * B * L * N * 2 + 3 * B * H * L * P * 2 + 3 * B * L * H * 2
                  + B * L * Nr * 4 + B * H * (L // 16) * Nr * 4 + B * H * (L // cfg.chunk) * Nr * 4
                  + B * H * P * N * 4 + B * H * (N + P + Nr) * 4)
    scan_flops = B * H * L * 2 * (2 * N * P + cfg.chunk * N + cfg.chunk * P)
    if args.leg in ("all", "scan", "bwd"):
        kraw, kc, phi_full = scan_inputs(m3, params16, cfg, u, torch)
        ka = dict(kc, phi=phi_full)
        if args.leg in ("all", "scan"):
            scan = lambda: K.siso_forward_raw(**kraw, chunk=128)  # noqa: E731
            scan_c = lambda: K.siso_forward(**kc, chunk=128)  # noqa: E731
            scan_r = lambda: K.siso_forward(**ka, chunk=128)  # noqa: E731
            # a kernel-boundary micro-measurement: enough launches that the clocks have
            # settled (a few ms of warmup), whatever --steps says for the headline; the
            # three forms alternate, and each keeps the better of its two averages
            for _ in range(max(args.warmup, 10)):
                scan()
                scan_c()
                scan_r()
            n = max(args.steps, 50)
            times = [(gpu_time_ms(scan, n, torch), gpu_time_ms(scan_c, n, torch),
                      gpu_time_ms(scan_r, n, torch)) for _ in range(2)]
            scan_ms = min(t[0] for t in times)
            comp_ms = min(t[1] for t in times)
            read_ms = min(t[2] for t in times)
            scan_gbs = scan_bytes / (scan_ms * 1e-3) / 1e9
            scan_tflops = scan_flops / (scan_ms * 1e-3) / 1e12
            line.update(scan_kernel_ms=round(scan_ms, 4),
                        scan_kernel_tok_s=round(tokens / (scan_ms * 1e-3), 1),
                        scan_kernel_gbs=round(scan_gbs, 1),
                        scan_kernel_tflops=round(scan_tflops, 2),
                        scan_kernel_mfma_frac=round(scan_tflops / BF16_PEAK_TFLOPS, 5),
                        scan_kernel_phi_compact_ms=round(comp_ms, 4),
                        scan_kernel_phi_compact_gbs=round(scan_compact_bytes / (comp_ms * 1e-3) / 1e9, 1),
                        scan_kernel_phi_read_ms=round(read_ms, 4),
                        scan_kernel_phi_read_gbs=round(scan_read_bytes / (read_ms * 1e-3) / 1e9, 1))
            line["roofline"] = {
                "kernel": "fwd_bf16_kernel<128,128,64,1,true> (m3s_fwd in raw mode, kernel "
                          "boundary: the preprocess and the phi carry inside the scan)",
                "bound": "hbm", "achieved": round(scan_gbs, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(scan_gbs / HBM_PEAK_GBS, 4),
                "traffic": traffic_figure("fwd_bf16_kernel_raw"),
                "traffic_source": TRAFFIC_SOURCE, "algorithmic_bytes": scan_bytes,
                "mfma_frac": round(scan_tflops / BF16_PEAK_TFLOPS, 5),
                "mfma_busy": counter_figure("fwd_bf16_kernel_raw", "mfma_busy_frac"),
                "mfma_busy_source": COUNTER_SOURCE,
                # the same scan fed by the preprocess launches, phi compact or materialised
                "phi_compact_frac": round(scan_compact_bytes / (comp_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "phi_read_frac": round(scan_read_bytes / (read_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if args.leg in ("all", "bwd"):
            # the training path's pair: with gradients the layer materialises phi and both
            # scans read it (phi_in_kernel=None)
            kr = dict(ka, phi=phi_full)
            with torch.no_grad():
                y, fs, fk, fv, res = K.siso_forward(**kr, chunk=128, save_residuals=True)
                dyk = torch.randn(y.shape, generator=gen.manual_seed(2), device=dev
                                  ).to(torch.bfloat16)
                bw = lambda: K.siso_backward_kernel(  # noqa: E731
                    dyk, res.ybar, kr["z"], kr["q"], kr["k"], kr["v"], kr["adt"], kr["gamma"],
                    kr["scale"], kr["phi"], kr["q_bias"], kr["k_bias"], res.chunk_states,
                    d_skip=kr["d_skip"], chunk=128)
                for _ in range(max(3, args.warmup)):
                    bw()
                bwd_ms = gpu_time_ms(bw, max(10, args.steps // 2), torch)
            bwd_flops = B * H * L * (2 * cfg.chunk * (3 * N + 2 * P) + 8 * P * N)
            # The backward's necessary bytes (no per-head rows): reads q, k (head-shared),
            # v, z, dy, ybar bf16, adt/gamma/scale f32, phi f32, the chunk states
            # bf16; writes dv, dz bf16, dadt/dqk/dscale/uw f32, dphi f32, dq/dk f32.
            nc = L // cfg.chunk
            bwd_bytes = (2 * B * L * N * 2 + 4 * B * H * L * P * 2
                         + 3 * B * H * L * 4 + phi_read + B * H * nc * N * P * 2
                         + 2 * B * H * L * P * 2 + 4 * B * H * L * 4 + B * H * L * Nr * 4
                         + 2 * B * L * N * 4)
            bwd_gbs = bwd_bytes / (bwd_ms * 1e-3) / 1e9
            line.update(bwd_kernel_ms=round(bwd_ms, 4),
                        bwd_kernel_tflops=round(bwd_flops / (bwd_ms * 1e-3) / 1e12, 2))
            line["bwd_roofline"] = {
                "kernel": "bwd_bf16_kernel<128,128,64,false> + headsum_kernel (m3s_bwd, phi "
                          "read: the training path's backward)",
                "bound": "hbm", "achieved": round(bwd_gbs, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(bwd_gbs / HBM_PEAK_GBS, 4),
                "algorithmic_bytes": bwd_bytes,
                "traffic": _sum_or_none(traffic_figure("bwd_bf16_kernel"),
                                        traffic_figure("headsum_kernel")),
                "traffic_source": TRAFFIC_SOURCE.replace("--leg scan", "--leg bwd"),
                "mfma_frac": round(bwd_flops / (bwd_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 5),
                "mfma_busy": counter_figure("bwd_bf16_kernel", "mfma_busy_frac"),
                "mfma_busy_source": COUNTER_SOURCE.replace("--leg scan", "--leg bwd")}
            del y, res, dyk, kr
        del ka, kc, kraw, phi_full
        torch.cuda.empty_cache()
        if args.leg != "all":
            print(json.dumps({"leg": args.leg, **line}))
            return

    # ---------------- decode ---------------------------------------------
    BD, T = 256, args.decode_tokens

    def rnd(shape, seed, scale=1.0):
        return torch.randn(*shape, generator=gen.manual_seed(seed), device=dev) * scale

    state = m3.SISOState(rnd((BD, H, P, N), 3, 0.1), rnd((BD, H, N), 4), rnd((BD, H, P), 5),
                         torch.rand(BD, H, Nr, generator=gen.manual_seed(6), device=dev) * 2 * math.pi)
    with torch.no_grad():
        q1 = torch.randn(BD, N, device=dev).to(torch.bfloat16)
        v1 = torch.randn(BD, H, P, device=dev).to(torch.bfloat16)
        s1 = torch.full((BD, H), 0.01, device=dev)
        ang1 = torch.randn(BD, Nr, device=dev)
        dstep = lambda: K.decode_step(q1, q1, v1, -s1, s1, s1 * 50, ang1,  # noqa: E731
                                      params16.c_bias.float(), params16.b_bias.float(), state,
                                      params16.d_skip.float(), v1)
        for _ in range(args.warmup):
            dstep()
        dec_kernel_ms = gpu_time_ms(dstep, 50, torch)
    dec_bytes = (2 * BD * H * P * N * 4 + 2 * BD * H * (N + P + Nr) * 4
                 + BD * N * 2 * 2 + 3 * BD * H * P * 2 + 3 * BD * H * 4 + BD * Nr * 4)
    dec_gbs = dec_bytes / (dec_kernel_ms * 1e-3) / 1e9
    line.update(decode_kernel_ms=round(dec_kernel_ms, 4), decode_kernel_gbs=round(dec_gbs, 1),
                decode_kernel_hbm_frac=round(dec_gbs / HBM_PEAK_GBS, 4),
                decode_kernel_bytes=dec_bytes,
                decode_kernel_traffic=traffic_figure("decode_kernel"))
    # a known-length run (kernel_decode.py:474-533): T steps in one m3s_decode_scan launch
    for bs in (BD, 1):
        with torch.no_grad():
            qs = torch.randn(bs, T, N, device=dev).to(torch.bfloat16)
            ks = torch.randn(bs, T, N, device=dev).to(torch.bfloat16)
            vs = torch.randn(bs, H, T, P, device=dev).to(torch.bfloat16)
            zs = torch.randn(bs, H, T, P, device=dev).to(torch.bfloat16)
            ss = torch.full((bs, H, T), 0.01, device=dev)
            ns, ls = -ss, ss * 50
            angs = torch.randn(bs, T, Nr, device=dev)
            cb, bb, dk = (params16.c_bias.float(), params16.b_bias.float(),
                          params16.d_skip.float())
            st_s = m3.SISOState(*(t[:bs].clone() for t in state))
            sscan = lambda: K.decode_scan(qs, ks, vs, ns, ss, ls, angs, cb, bb, st_s,  # noqa: E731
                                          dk, zs)
            sscan()
            scan_ms = gpu_time_ms(sscan, 5 if bs == BD else 20, torch)
        line[f"decode_scan_ms_per_token_b{bs}"] = round(scan_ms / T, 5)
        del qs, ks, vs, zs, ss, ns, ls, angs, st_s
    line["decode_scan_tokens"] = T
    if args.leg == "decode":
        print(json.dumps({"leg": "decode", **line}))
        return
    toks = [rnd((BD, DM), 1000 + t).to(torch.bfloat16) for t in range(T)]
    with torch.no_grad():
        for t in range(4):
            _, state = m3.mamba3_siso_decode_step(params16, toks[t], cfg, state)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for t in range(T):
            _, state = m3.mamba3_siso_decode_step(params16, toks[t], cfg, state)
        torch.cuda.synchronize()
        dec_ms = (time.perf_counter() - t0) * 1e3 / T
    # the configs[3] layer step's necessary bytes: the token rows in and out, both
    # projection weights, the in_proj row written and read, the state read and written,
    # the gated y written and read
    d_in = cfg.d_in_proj
    dec_layer_bytes = (BD * DM * 2 * 2 + (DM * d_in + cfg.d_inner * DM) * 2 + BD * d_in * 2 * 2
                       + 2 * BD * H * P * N * 4 + 2 * BD * H * (N + P + Nr) * 4
                       + BD * cfg.d_inner * 2 * 2)
    line.update(decode_layer_bytes=dec_layer_bytes,
                decode_layer_gbs=round(dec_layer_bytes / (dec_ms * 1e-3) / 1e9, 1),
                decode_layer_hbm_frac=round(dec_layer_bytes / (dec_ms * 1e-3) / 1e9
                                            / HBM_PEAK_GBS, 4))
    # The legs from here to the headline run back to back, without emptying the allocator
    # cache in between: the GPU lowers its clocks within a millisecond or two of idling
    # (measured: a 20 ms pause before 5 warmup steps costs the next 20 forwards 7%, an
    # empty_cache() after the fwd+bwd leg 3.5%), so a pause would put the timed steps on
    # the ramp back up instead of the steady state a busy device runs at.
    del toks, state

    # ---------------- forward + backward ---------------------------------
    pg = m3.SISOParams(*(t.detach().clone().requires_grad_(True) for t in params32))
    ug = u.detach().clone().requires_grad_(True)
    dy = torch.randn(B, L, DM, generator=gen.manual_seed(2), device=dev).to(torch.bfloat16)

    def fwdbwd_step():
        # the gradients of u and of every parameter, returned (as jax.grad does) rather
        # than accumulated into .grad, which would add one add kernel per tensor
        y, _ = m3.mamba3_siso_layer(pg, ug, cfg)
        return torch.autograd.grad(y, (ug, *pg), dy)

    for _ in range(max(3, args.warmup)):
        fwdbwd_step()
    fb_iters = max(3, args.steps // 4)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(fb_iters):
        fwdbwd_step()
    torch.cuda.synchronize()
    fb_ms = (time.perf_counter() - t0) * 1e3 / fb_iters
    del pg, ug, dy

    # ---------------- headline: layer forward, the K timed steps ----------
    def fwd_step():
        with torch.no_grad():
            return m3.mamba3_siso_layer(params16, u, cfg)

    for _ in range(args.warmup):
        fwd_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        fwd_step()
    torch.cuda.synchronize()
    fwd_ms = (time.perf_counter() - t0) * 1e3 / args.steps

    lm = None if args.no_lm else lm_legs(m3, torch, dev)

    # ---------------- CPU baseline: the oracle on a bounded sample --------------------
    cpu_base = None
    if not args.no_cpu_baseline:
        cpu_base = cpu_baseline(m3, params32, cfg, torch)

    out = {
        "metric": METRIC,
        "value": round(tokens / (fwd_ms * 1e-3), 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(fwd_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs, init_params(seed=0) weights)",
        "config": {"workload": "configs[1]: one Mamba-3 SISO layer forward (in_proj; BCNorm "
                               "with the rotary table; the HIP chunked scan reading the raw "
                               "dt / a / trap slices; out_proj)",
                   "batch": B, "seq_len": L, "nheads": H, "headdim": P, "d_state": N,
                   "d_model": DM, "chunk": 128, "n_angles": Nr},
        "gemm_solutions": "recorded (mamba3-siso-tpu_amd/tuned_gemms.csv)" if tuned
                          else "hipBLASLt default heuristic",
        "fwd_bwd_ms": round(fb_ms, 3),
        "fwd_bwd_tok_s": round(tokens / (fb_ms * 1e-3), 1),
        "decode_ms_per_token": round(dec_ms, 4),
        **{k: v for k, v in line.items() if k != "roofline"},
        "layer_roofline": layer_roofline(B, L, DM, cfg, scan_bytes, scan_flops, fwd_ms),
        "lm": lm,
        "reference_tpu_v5e": {"fwd_kernel_ms_chunk128_pinned": 21.66, "fwd_bwd_ms": 80.1,
                              "decode_ms_per_token_b256": 1.4},
        "roofline": line["roofline"],
        "cpu_baseline": cpu_base,
    }
    print(json.dumps(out))


def lm_legs(m3, torch, dev):
    """the 8-layer byte LM (d_model 768, headdim 64, d_state 128,
    chunk 128, gated MLP 1536, vocab 256, tied head; 59.1M parameters) trained on B=16 x
    L=2048 windows of i.i.d. Zipf(1.1) bytes, bf16 products, float32 master weights,
    clip 1.0 + AdamW (wd 0.1, warmup-cosine lr). tok/s over steps 10-60 (batches staged on
    the device beforehand). Then the decode stack on the same model: one recorded decode
    step per token (batch 1 and batch 256), and `generate` end to end (sampling included)."""
    T = m3.train
    scfg = m3.SISOConfig(d_model=768, d_state=128, headdim=64, expand=2, chunk=128,
                         policy_name="bf16")
    cfg = m3.model.LMConfig(vocab_size=256, n_layers=8, siso=scfg, tie_head=True,
                            d_intermediate=1536)
    bsz, seqlen = 16, 2048
    params = T.train_params(m3.model.init_lm(cfg, 0, device=dev))
    data = T.zipf_bytes(8 << 20, s=1.1, seed=0)
    stream = T.batches(data, bsz, seqlen, seed=1, device=dev)
    staged = [next(stream) for _ in range(60)]
    opt = T.make_optimizer(params, lr=1e-3, warmup=100, steps=2000)
    step = T.make_step(cfg, opt)
    losses = []
    for i in range(10):
        loss, params, opt = step(params, opt, *staged[i])
        losses.append(loss)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(10, 60):
        loss, params, opt = step(params, opt, *staged[i])
        losses.append(loss)
    torch.cuda.synchronize()
    train_s = time.perf_counter() - t0
    out = {"workload": "configs[4]: 8-layer byte LM training step (B=16, L=2048)",
           "params": cfg.param_count(),
           "train_tok_s": round(50 * bsz * seqlen / train_s, 1),
           "train_ms_per_step": round(train_s * 1e3 / 50, 3),
           "loss_step0": round(float(losses[0]), 4), "loss_step59": round(float(losses[-1]), 4),
           "zipf_entropy_nats": round(float(_zipf_entropy(1.1)), 4)}
    del staged, opt, stream
    torch.cuda.empty_cache()

    dp = m3.model.decode_params(params, cfg)
    for batch in (1, 256):
        dg = T.DecodeGraph(dp, cfg, batch=batch)
        tok = torch.randint(0, 256, (batch,), device=dev)
        for _ in range(5):
            dg.step(tok)
        ms = gpu_time_ms(lambda: dg.step(tok), 200, torch)
        out[f"decode_graph_ms_per_token_b{batch}"] = round(ms, 4)
        del dg
    T.generate(dp, cfg, 0, [104, 105], n_tokens=8)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ids = T.generate(dp, cfg, 0, list(b"the "), n_tokens=256)
    torch.cuda.synchronize()
    out["generate_ms_per_token_b1"] = round((time.perf_counter() - t0) * 1e3 / 256, 4)
    assert len(ids) == 4 + 256
    return out


def _zipf_entropy(s):
    p = [(v + 1) ** -s for v in range(256)]
    z = sum(p)
    return -sum(x / z * math.log(x / z) for x in p)


TRAFFIC_SOURCE = ("profiles/traffic.json: rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, of "
                  "`bench.py --leg scan`, each scaled by its ratio on `bench.py --leg copy`; "
                  "measured in its own runs, not in this one")


COUNTER_SOURCE = ("profiles/sq_counters.json: rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES "
                  "GRBM_GUI_ACTIVE (with six other SQ counters) of `bench.py --leg scan`: MFMA "
                  "busy cycles over 1024 SIMDs x GPU-active cycles per XCD; measured in its own "
                  "runs, not in this one")


def _sum_or_none(*xs):
    return None if any(x is None for x in xs) else sum(xs)


def counter_figure(kernel, field):
    """One figure of ``kernel`` from the committed SQ counter summary
    (profiles/sq_counters.json), or None if absent."""
    try:
        with open(os.path.join(ROOT, "profiles", "sq_counters.json")) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    return rec.get("kernels", {}).get(kernel, {}).get(field)


def traffic_figure(kernel):
    """HBM bytes per launch of ``kernel`` from the committed counter summary
    (profiles/traffic.json: FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the
    ratio the same counter shows for a plain 1 GiB copy), or None if absent."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    k = rec.get("kernels", {}).get(kernel)
    return None if k is None else k.get("traffic_bytes")


def cpu_baseline(m3, params32, cfg, torch):
    """The CPU oracle (torch, float32) running the same layer forward on one sequence of
    the workload, repeated until ~10 s of CPU work; reported, never a gate."""
    from oracle import siso_oracle as O

    threads = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(threads)
    pd = {f: getattr(params32, f).detach().float().cpu() for f in params32._fields}
    g = torch.Generator().manual_seed(0)
    u = torch.randn(1, 8192, cfg.d_model, generator=g).to(torch.bfloat16).float()
    reps, t_total = 0, 0.0
    with torch.no_grad():
        while t_total < 10.0 and reps < 20:
            t0 = time.perf_counter()
            O.layer_forward(pd, u, d_state=cfg.d_state, headdim=cfg.headdim, expand=cfg.expand,
                            chunk=cfg.chunk)
            t_total += time.perf_counter() - t0
            reps += 1
    return {"value": round(reps * u.shape[1] / t_total, 1), "unit": "tok/s",
            "cores": os.cpu_count(), "threads": torch.get_num_threads(), "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": f"{reps} x one sequence (B=1, L=8192, d_model=1024) of the configs[1] layer "
                      f"forward through oracle.siso_oracle.layer_forward in float32 on "
                      f"{platform.processor() or platform.machine()}"}


def _cpu_model() -> str:
    """The host CPU's model name (Linux /proc/cpuinfo), or the platform string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


if __name__ == "__main__":
    main()
