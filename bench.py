"""Benchmark of the fused 2D FNO spectral block on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 50] [--workload c2]

Workload (default): the 256^2 Navier-Stokes-like block
    y = GELU(SpectralConv(x) + Ws x),  x [32, 64, 256, 256] fp32 Gaussian random
    field, n_modes (64, 64) -> 64 rows x 33 rfft columns, dense complex weight
    W [64, 64, 64, 33] (re/im ~ N(0, 1/4096)), 1x1 skip Ws [64, 64] ~ N(0, 1/64),
    bias 0, exact erf GELU.
One step = one call of the block on one batch already resident in HBM.

Prints ONE JSON line: value = achieved algorithmic HBM bandwidth (read x once,
write y once, read W/Ws/bias once) over the timed steps, in GB/s; plus
us_per_call, the roofline of the block, the torch.fft + einsum ROCm path
timed on the same GPU, and the CPU baseline (the oracle restatement on the
host cores, bounded sample).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch
import torch.nn.functional as F

HBM_PEAK_GBS = 8000.0
METRIC = "µs/call + achieved HBM GB/s, fused 2D spectral block B32 C64 256² fp32"

WORKLOADS = {
    # name: (B, C, H, W, n_modes)
    "c2": (32, 64, 256, 256, (64, 64)),
    "c2_32": (32, 64, 256, 256, (32, 32)),
    "c1": (32, 64, 128, 128, (32, 32)),
    # a non-power-of-two grid (the Darcy-flow resolution of the FNO paper):
    # the generic path, pruned direct DFTs on both axes
    "darcy421": (16, 32, 421, 421, (32, 32)),
}


# Workloads timed through the nn.Module API (one forward per step)
MODULE_WORKLOADS = {
    "c0": "1D SpectralConv x[16,64,1024] ~N(0,1), n_modes 30 -> 16 rfft modes, dense W[64,64,16]",
    "c3": "4-layer FNO forward x[64,1,256,256] bf16 GRF (+2 grid channels), lifting 3->128->64, "
          "4 blocks hidden 64 n_modes (64,64) with channel MLP 64->32->64 and soft-gating, "
          "projection 64->128->1",
    "c4": "3D TFNO block x[8,32,64,64,64] GRF, Tucker rank 0.1 spectral conv n_modes (16,16,16) "
          "-> 16x16x9 modes (factorized), 1x1 skip, bias, erf GELU",
}


PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def profiled_traffic(workload):
    """HBM bytes per block call measured with rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE passes over this script, each scaled by what the counter reads
    for a plain 1 GiB device copy (see the profile's calibration table), summed
    over the block's kernels; None when no such profile is committed."""
    B, C, H, W, nm = WORKLOADS[workload]
    m1, m2h = nm[0], nm[1] // 2 + 1
    stem = os.path.join(PROFILES, f"fused2d_block_b{B}c{C}_{H}x{W}_m{m1}x{m2h}")
    for path in (stem + "_traffic.md", stem + ".md"):
        try:
            with open(path) as f:
                for line in f:
                    if line.startswith("traffic_bytes_per_call:"):
                        return int(line.split(":", 1)[1].strip().replace(",", ""))
        except OSError:
            pass
    return None


def algorithmic_bytes(B, C, H, W, m1, m2h):
    x = B * C * H * W * 4
    w = C * C * m1 * m2h * 8
    return 2 * x + w + C * C * 4 + C * 4


def make_inputs(B, C, H, W, nm, device):
    from neuraloperator_amd.synthetic import gaussian_random_field
    m1, m2h = nm[0], nm[1] // 2 + 1
    x = gaussian_random_field((B, C, H, W), seed=2024, device=device)
    g = torch.Generator().manual_seed(7)
    w = torch.complex(torch.randn(C, C, m1, m2h, generator=g),
                      torch.randn(C, C, m1, m2h, generator=g)) / 64.0
    ws = torch.randn(C, C, generator=g) / 8.0
    bias = torch.zeros(C)
    return x, w.to(device), ws.to(device), bias.to(device), (m1, m2h)


def torch_rocm_block(x, w, bias, ws, m1, m2h):
    """The reference op sequence (rfftn, fftshift, window, einsum, ifftshift,
    ifftn, Hermitian fix-up, irfft, bias) + skip + GELU in torch on the GPU."""
    B, C, H, W = x.shape
    X = torch.fft.fftshift(torch.fft.rfftn(x, norm="forward", dim=(-2, -1)), dim=(-2,))
    out = torch.zeros(B, w.shape[1], H, W // 2 + 1, dtype=torch.complex64, device=x.device)
    r0 = H // 2 - m1 // 2
    out[:, :, r0:r0 + m1, :m2h] = torch.einsum("bixy,ioxy->boxy", X[:, :, r0:r0 + m1, :m2h], w)
    out = torch.fft.ifftn(torch.fft.ifftshift(out, dim=(-2,)), s=(H,), dim=(-2,), norm="forward")
    out[..., 0].imag.zero_()
    out[..., -1].imag.zero_()
    y = torch.fft.irfft(out, n=W, dim=-1, norm="forward") + bias.view(1, -1, 1, 1)
    y = y + torch.einsum("oi,bihw->bohw", ws, x)
    return F.gelu(y)


def event_times(fn, iters, stream, flush=None):
    """Per-call durations (ms) with HIP events on ``stream``; optional cache
    flush between calls, outside the timed interval."""
    out = []
    for _ in range(iters):
        if flush is not None:
            flush()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        fn()
        e1.record(stream)
        e1.synchronize()
        out.append(e0.elapsed_time(e1))
    return out


def timed_region(step, warmup, steps, stream):
    """W untimed warm-up steps, then exactly K timed steps bracketed by
    synchronisations.  Returns (wall ms per step, HIP-event µs per step): the
    events sit on the launch stream at both ends of the same K back-to-back
    calls, so both figures describe the same region."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return (t1 - t0) * 1e3 / steps, e0.elapsed_time(e1) * 1e3 / steps


N_WARM_EXTRA, N_EVENT_CALLS = 10, 50


def per_call_medians(step, stream, dev):
    """Median µs of single calls timed with HIP events: warm (calls back to
    back, 10 warm-ups then 50 calls) and cold (a 1 GiB scratch write before
    each of 50 calls evicts the 256 MB Infinity Cache)."""
    for _ in range(N_WARM_EXTRA):
        step()
    warm = event_times(step, N_EVENT_CALLS, stream)
    scratch = torch.empty(1 << 28, dtype=torch.float32, device=dev)
    cold = event_times(step, N_EVENT_CALLS, stream, flush=lambda: scratch.fill_(1.0))
    del scratch
    return statistics.median(warm) * 1e3, statistics.median(cold) * 1e3


def graph_us_per_call(step, stream, calls=20, replays=10):
    """µs per call of `calls` forward calls captured in one HIP graph and
    replayed back to back (the same kernels, without the host launch path);
    None when the step cannot be captured."""
    try:
        for _ in range(3):
            step()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(calls):
                step()
        g.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        cur = torch.cuda.current_stream()
        e0.record(cur)
        for _ in range(replays):
            g.replay()
        e1.record(cur)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (calls * replays)
    except RuntimeError:
        return None


def cpu_baseline(B, C, H, W, nm, total_bytes, budget_s=20.0):
    """The oracle (plain-torch restatement of the reference forward) on the
    host cores, on a bounded sample of the batch."""
    from oracle import spectral_ref as R
    torch.set_num_threads(os.cpu_count() or 1)
    from neuraloperator_amd.synthetic import gaussian_random_field
    m1, m2h = nm[0], nm[1] // 2 + 1
    bs = 1
    x = gaussian_random_field((bs, C, H, W), seed=5)
    g = torch.Generator().manual_seed(6)
    w = torch.complex(torch.randn(C, C, m1, m2h, generator=g), torch.randn(C, C, m1, m2h, generator=g)) / 64
    ws = torch.randn(C, C, generator=g) / 8
    bias = torch.zeros(C, 1, 1)

    def run():
        y = R.spectral_conv_forward(x, w, bias, [m1, m2h], [m1, m2h])
        return R.gelu(y + R.linear_skip(x, ws))

    for _ in range(2):
        run()
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < budget_s and len(times) < 50):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > 3 * budget_s:
            break
    per_sample = statistics.median(times)
    per_call = per_sample * B / bs
    return {
        "value": round(total_bytes / per_call / 1e9, 3),
        "unit": "GB/s",
        "us_per_call": round(per_call * 1e6, 1),
        "cores": torch.get_num_threads(),
        "os_cpu_count": os.cpu_count(),
        "kind": "port",
        "sample": f"{bs} of {B} samples, median of {len(times)} runs after 2 warm-ups, "
                  f"scaled x{B // bs} to one call",
    }


def _oracle_layer(blocks, i):
    """Parameters of FNOBlocks layer i as float64 CPU tensors for the oracle."""
    conv = blocks.convs[i]
    d = lambda t: t.detach().cpu().double()
    layer = {"conv": dict(weight=conv.weight.to_tensor().detach().cpu().to(torch.complex128),
                          bias=d(conv.bias), n_modes=conv.n_modes, max_n_modes=conv.max_n_modes),
             "fno_skip": {"type": "linear", "w": d(blocks.fno_skips[i].conv.weight)[:, :, 0]}}
    if blocks.use_channel_mlp:
        m = blocks.channel_mlp[i]
        layer["mlp"] = {"weights": [d(f.weight) for f in m.fcs], "biases": [d(f.bias) for f in m.fcs]}
        layer["mlp_skip"] = {"type": "soft-gating", "w": d(blocks.channel_mlp_skips[i].weight)}
    return layer


C4_TUCKER_RANK = (20, 20, 10, 10, 6)   # what rank=0.1 gives for the (32, 32, 16, 16, 9) weight


def torch_rocm_conv1d(x, w, bias, m):
    """The reference op sequence of a 1D SpectralConv in torch on the GPU:
    rfft(norm="forward"), first m bins, einsum, zero-padded irfft, bias."""
    B, _, N = x.shape
    X = torch.fft.rfft(x, norm="forward")
    out = torch.zeros(B, w.shape[1], N // 2 + 1, dtype=torch.complex64, device=x.device)
    out[..., :m] = torch.einsum("bix,iox->box", X[..., :m], w)
    return torch.fft.irfft(out, n=N, norm="forward") + bias.view(1, -1, 1)


def torch_rocm_tucker3d(x, core, factors, bias, ws, m):
    """The reference's factorized Tucker 3D SpectralConv + 1x1 skip + GELU in
    torch on the GPU: rfftn, fftshift, centred window, the Tucker chain as
    pairwise einsums (input factor, core with the mode factors, output
    factor), ifftshift, ifftn over the first two axes, Hermitian fix-up,
    irfft, bias."""
    B, C, D1, D2, D3 = x.shape
    m1, m2, m3 = m
    X = torch.fft.fftshift(torch.fft.rfftn(x, norm="forward", dim=(-3, -2, -1)), dim=(-3, -2))
    r1, r2 = D1 // 2 - m1 // 2, D2 // 2 - m2 // 2
    Xw = X[:, :, r1:r1 + m1, r2:r2 + m2, :m3]
    Uin, Uout, U1, U2, U3 = factors
    K = torch.einsum("ghabc,xa->ghxbc", core, U1)
    K = torch.einsum("ghxbc,yb->ghxyc", K, U2)
    K = torch.einsum("ghxyc,zc->ghxyz", K, U3)
    t = torch.einsum("bixyz,ig->bgxyz", Xw, Uin)
    t = torch.einsum("bgxyz,ghxyz->bhxyz", t, K)
    Y = torch.einsum("bhxyz,oh->boxyz", t, Uout)
    out = torch.zeros(B, Y.shape[1], D1, D2, D3 // 2 + 1, dtype=torch.complex64, device=x.device)
    out[:, :, r1:r1 + m1, r2:r2 + m2, :m3] = Y
    out = torch.fft.ifftn(torch.fft.ifftshift(out, dim=(-3, -2)), s=(D1, D2), dim=(-3, -2),
                          norm="forward")
    out[..., 0].imag.zero_()
    out[..., -1].imag.zero_()
    y = torch.fft.irfft(out, n=D3, dim=-1, norm="forward") + bias.view(1, -1, 1, 1, 1)
    y = y + F.conv1d(x.reshape(B, C, -1), ws.view(ws.shape[0], C, 1)).view_as(y)
    return F.gelu(y)


def _torch_mlp(m, x):
    """ChannelMLP (two 1x1 Conv1d with GELU between) in torch."""
    B, C, *S = x.shape
    h = x.reshape(B, C, -1)
    fc0, fc1 = m.fcs
    h = F.gelu(F.conv1d(h, fc0.weight, fc0.bias))
    h = F.conv1d(h, fc1.weight, fc1.bias)
    return h.reshape(B, h.shape[1], *S)


def torch_rocm_fno(model, x):
    """The reference FNO forward (grid embedding, lifting, blocks with
    spectral conv + linear skip + GELU, channel MLP + soft-gating + GELU, no
    activations in the last layer, projection) in torch on the GPU, 1x1
    layers as Conv1d."""
    B, _, H, W = x.shape
    gx = torch.linspace(0, 1, H + 1, device=x.device)[:-1]
    gy = torch.linspace(0, 1, W + 1, device=x.device)[:-1]
    g0, g1 = torch.meshgrid(gx, gy, indexing="ij")
    h = torch.cat([x, g0.expand(B, 1, H, W), g1.expand(B, 1, H, W)], dim=1)
    h = _torch_mlp(model.lifting, h)
    blk = model.fno_blocks
    for i in range(blk.n_layers):
        conv = blk.convs[i]
        w = conv.weight.to_tensor()
        m1, m2h = w.shape[2], w.shape[3]
        Cc = h.shape[1]
        X = torch.fft.fftshift(torch.fft.rfftn(h.float(), norm="forward", dim=(-2, -1)), dim=(-2,))
        out = torch.zeros(B, w.shape[1], H, W // 2 + 1, dtype=torch.complex64, device=x.device)
        r0 = H // 2 - m1 // 2
        out[:, :, r0:r0 + m1, :m2h] = torch.einsum("bixy,ioxy->boxy", X[:, :, r0:r0 + m1, :m2h], w)
        out = torch.fft.ifftn(torch.fft.ifftshift(out, dim=(-2,)), s=(H,), dim=(-2,), norm="forward")
        out[..., 0].imag.zero_()
        out[..., -1].imag.zero_()
        spec = torch.fft.irfft(out, n=W, dim=-1, norm="forward") + conv.bias.view(1, -1, 1, 1)
        sk = F.conv1d(h.reshape(B, Cc, -1), blk.fno_skips[i].conv.weight).view(B, -1, H, W)
        gate = blk.channel_mlp_skips[i].weight * h
        last = i == blk.n_layers - 1
        h = spec + sk
        if not last:
            h = F.gelu(h)
        h = _torch_mlp(blk.channel_mlp[i], h) + gate
        if not last:
            h = F.gelu(h)
    return _torch_mlp(model.projection, h)


def module_workload(name, dev):
    """The workloads timed through the module API: a dict with the step
    function, algorithmic bytes, dtype, the CPU-baseline runner, the torch
    ROCm path of the same computation and extra config entries."""
    import neuraloperator_amd as na
    from neuraloperator_amd import _native as nat
    from neuraloperator_amd.synthetic import gaussian_random_field
    torch.manual_seed(7)
    if name == "c0":
        B, C, N = 16, 64, 1024
        conv = na.SpectralConv(C, C, (30,)).to(dev)            # 30 // 2 + 1 = 16 modes
        g = torch.Generator().manual_seed(7)
        with torch.no_grad():
            w = torch.complex(torch.randn(C, C, 16, generator=g), torch.randn(C, C, 16, generator=g)) / 64
            conv.weight.tensor.copy_(w.to(dev))
        x = torch.randn(B, C, N, generator=g).to(dev)
        nbytes = 2 * B * C * N * 4 + C * C * 16 * 8 + C * 4

        def cpu():
            from oracle import spectral_ref as R
            xc = x.cpu()
            return lambda: R.spectral_conv_forward(
                xc, conv.weight.to_tensor().detach().cpu(), conv.bias.detach().cpu(), conv.n_modes,
                conv.max_n_modes), B, B
        wt = conv.weight.to_tensor().detach()
        return dict(step=lambda: conv(x), nbytes=nbytes, dtype="f32", cpu=cpu, graph=True,
                    rocm=(lambda: torch_rocm_conv1d(x, wt, conv.bias.detach(), 16),
                          "torch.fft.rfft + einsum + irfft + bias (rocFFT, rocBLAS), same GPU"),
                    extra={"batch": B, "channels": C, "N": N, "modes": [16]})
    if name == "c4":
        B, C, S = 8, 32, 64
        conv = na.SpectralConv(C, C, (16, 16, 16), factorization="Tucker", rank=0.1,
                               implementation="factorized").to(dev)
        if tuple(conv.weight.rank) != C4_TUCKER_RANK:
            raise RuntimeError(f"Tucker rank {conv.weight.rank} != recorded {C4_TUCKER_RANK}")
        x = gaussian_random_field((B, C, S, S, S), seed=2024, device=dev)
        ws = (torch.randn(C, C) / (C ** 0.5)).to(dev)
        nbytes = 2 * B * C * S ** 3 * 4 + C * C * 4 + C * 4 + sum(
            p.numel() * p.element_size() for p in conv.weight.parameters())

        def cpu():
            from oracle import spectral_ref as R
            xs = x[:1].cpu()
            core = conv.weight.core.detach().cpu()
            factors = [f.detach().cpu() for f in conv.weight.factors]
            wsc = ws.cpu()
            return lambda: R.gelu(R.spectral_conv_forward(
                xs, {"tucker": (core, factors)}, conv.bias.detach().cpu(), conv.n_modes,
                conv.max_n_modes, implementation="factorized") + R.linear_skip(xs, wsc)), 1, B
        core = conv.weight.core.detach()
        factors = [f.detach() for f in conv.weight.factors]
        return dict(step=lambda: conv._forward_hip(x, None, nat.SKIP_LINEAR, ws, nat.ACT_GELU),
                    nbytes=nbytes, dtype="f32", cpu=cpu,
                    rocm=(lambda: torch_rocm_tucker3d(x, core, factors, conv.bias.detach(), ws,
                                                      (16, 16, 9)),
                          "torch.fft.rfftn + Tucker einsum chain + ifftn/irfft + conv1d skip + "
                          "gelu (rocFFT, rocBLAS, MIOpen), same GPU"),
                    extra={"batch": B, "channels": C, "grid": [S, S, S], "modes": [16, 16, 9],
                           "tucker_rank": list(C4_TUCKER_RANK)})
    # c3
    B, H = 64, 256
    model = na.FNO((64, 64), in_channels=1, out_channels=1, hidden_channels=64, n_layers=4).to(dev)
    x = gaussian_random_field((B, 1, H, H), seed=2024, device=dev).to(torch.bfloat16)
    # per block: bf16 activation in and out, the block's weights once
    blk = model.fno_blocks
    wbytes = sum(p.numel() * p.element_size() for p in blk.parameters()) // blk.n_layers
    nbytes = blk.n_layers * (2 * B * 64 * H * H * 2 + wbytes)

    def cpu():
        from oracle import spectral_ref as R
        d = lambda t: t.detach().cpu().double()
        mlp = lambda m: {"weights": [d(f.weight) for f in m.fcs], "biases": [d(f.bias) for f in m.fcs]}
        params = {"lifting": mlp(model.lifting), "projection": mlp(model.projection),
                  "layers": [_oracle_layer(blk, i) for i in range(blk.n_layers)]}
        xs = x[:1].float().cpu().double()
        return lambda: R.fno_forward(xs, params), 1, B
    # bf16 mixed precision: under torch.autocast(bfloat16) the 1x1 layers
    # (lifting, channel MLPs, projection) take bf16-rounded operands with fp32
    # accumulation, and the activations between the lifting, the layers and
    # the projection are stored in bf16; the complex64 spectral path, the
    # skips and every accumulation are fp32 (the bf16 input is widened on
    # entry)
    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            return model(x.float())

    def rocm():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            return torch_rocm_fno(model, x.float())
    return dict(step=step, nbytes=nbytes,
                dtype="bf16 activation storage and 1x1-layer operands (autocast), fp32 "
                      "accumulation, complex64 spectral path",
                cpu=cpu,
                rocm=(rocm, "the same FNO forward in torch ops under the same autocast: "
                            "torch.fft + einsum + Conv1d + gelu (rocFFT, rocBLAS, MIOpen), same GPU"),
                extra={"batch": B, "grid": [H, H], "hidden": 64, "n_layers": 4, "modes": [64, 33]})


def bench_module(args):
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    wl = module_workload(args.workload, dev)
    step, nbytes, dtype, cpu, extra = wl["step"], wl["nbytes"], wl["dtype"], wl["cpu"], wl["extra"]
    rocm_fn, rocm_what = wl["rocm"] if wl.get("rocm") else (None, None)
    with torch.no_grad():
        ms_per_step, us_events = timed_region(step, args.warmup, args.steps, stream)
        us_warm, us_cold = per_call_medians(step, stream, dev)
        us_graph = graph_us_per_call(step, stream) if wl.get("graph") else None
    line = {
        "metric": f"µs/call + achieved HBM GB/s, {MODULE_WORKLOADS[args.workload]}",
        "value": round(nbytes / (ms_per_step * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "us_per_call": round(ms_per_step * 1e3, 1),
        "us_per_call_median_warm": round(us_warm, 1),
        "us_per_call_median_cold": round(us_cold, 1),
        "us_per_call_graph": None if us_graph is None else round(us_graph, 2),
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (seeded Gaussian random field / normal inputs, seeded random-init weights)",
        "config": {"workload": MODULE_WORKLOADS[args.workload], "algorithmic_bytes": nbytes,
                   **extra},
        "roofline": {"bound": "hbm", "achieved": round(nbytes / (us_events * 1e-6) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(nbytes / (us_events * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None, "us_per_call": round(us_events, 1),
                     "kernel": "whole forward; HIP events on the launch stream around the timed "
                               "steps, per call"},
    }
    if rocm_fn is not None and not args.no_torch:
        with torch.no_grad():
            for _ in range(2):
                rocm_fn()
            tt = event_times(rocm_fn, 5, stream)
        line["torch_rocm_baseline"] = {
            "us_per_call": round(statistics.median(tt) * 1e3, 1),
            "gbs": round(nbytes / (statistics.median(tt) * 1e-3) / 1e9, 1),
            "what": rocm_what}
    if not args.no_cpu:
        torch.set_num_threads(os.cpu_count() or 1)
        run, done, total = cpu()
        with torch.no_grad():
            run()
            times = []
            t_start = time.perf_counter()
            while len(times) < 3 or (time.perf_counter() - t_start < 20 and len(times) < 20):
                t1 = time.perf_counter()
                run()
                times.append(time.perf_counter() - t1)
        per_call = statistics.median(times) * total / done
        line["cpu_baseline"] = {"value": round(nbytes / per_call / 1e9, 3), "unit": "GB/s",
                                "us_per_call": round(per_call * 1e6, 1),
                                "cores": torch.get_num_threads(), "kind": "port",
                                "sample": f"{done} of {total} samples, median of {len(times)} runs, "
                                          f"scaled x{total // done} to one call"}
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # the GPU's clocks settle over the first tens of milliseconds of work:
    # 50 untimed calls (about 25 ms of the headline block) before the timed ones
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="c2", choices=sorted(WORKLOADS) + sorted(MODULE_WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-torch", action="store_true", help="skip the torch ROCm baseline")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU only; multi-GPU runs are not part "
                                   "of it (the block shards by batch with no communication)",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    if args.workload in MODULE_WORKLOADS:
        return bench_module(args)

    import neuraloperator_amd  # noqa: F401  (loads the library early)
    from neuraloperator_amd import _native as nat
    from neuraloperator_amd import functional as Fh

    dev = torch.device("cuda:0")
    B, C, H, W, nm = WORKLOADS[args.workload]
    x, w, ws, bias, (m1, m2h) = make_inputs(B, C, H, W, nm, dev)
    y = torch.empty_like(x)
    stream = torch.cuda.current_stream(dev)
    fused = Fh.spectral_block_is_fused(B, C, C, [H, W], [m1, m2h], nat.SKIP_LINEAR)
    total_bytes = algorithmic_bytes(B, C, H, W, m1, m2h)

    # preallocate the workspace once so the timed calls do not allocate
    lib = nat.load()
    sz, md = nat.i32_array([H, W]), nat.i32_array([m1, m2h])
    wsb = lib.fno_spectral_block_workspace_bytes(B, C, C, 2, sz, md)
    wsbuf = torch.empty(wsb, dtype=torch.uint8, device=dev)
    import ctypes
    P = lambda t: ctypes.c_void_p(t.data_ptr())

    def step():
        rc = lib.fno_spectral_block_f32(P(x), P(w), P(bias), P(ws), P(y), B, C, C, 2, sz, md, 1,
                                        nat.SKIP_LINEAR, nat.ACT_GELU, P(wsbuf), wsb,
                                        ctypes.c_void_p(stream.cuda_stream))
        if rc:
            raise RuntimeError(nat.last_error())

    ms_per_step, us_events = timed_region(step, args.warmup, args.steps, stream)
    us_warm, us_cold = per_call_medians(step, stream, dev)

    # device copy bandwidth as a calibration of what HBM delivers
    src = torch.empty(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    ct = event_times(lambda: dst.copy_(src), 10, stream)
    copy_gbs = 2 * src.numel() * 4 / (statistics.median(ct) * 1e-3) / 1e9
    del src, dst

    rocm = None
    if not args.no_torch:
        with torch.no_grad():
            fn = lambda: torch_rocm_block(x, w, bias, ws, m1, m2h)
            for _ in range(2):
                fn()
            tt = event_times(fn, 5, stream)
        rocm = {"us_per_call": round(statistics.median(tt) * 1e3, 1),
                "gbs": round(total_bytes / (statistics.median(tt) * 1e-3) / 1e9, 1),
                "what": "torch.fft (rocFFT) + einsum + irfft + conv + gelu, same GPU"}

    value = total_bytes / (ms_per_step * 1e-3) / 1e9
    achieved_block = total_bytes / (us_events * 1e-6) / 1e9
    line = {
        "metric": METRIC if args.workload == "c2" else
                  f"µs/call + achieved HBM GB/s, fused 2D spectral block B{B} C{C} {H}x{W} "
                  f"modes {m1}x{m2h} fp32",
        "value": round(value, 1),
        "unit": "GB/s",
        "us_per_call": round(ms_per_step * 1e3, 1),
        "us_per_call_median_warm": round(us_warm, 1),
        "us_per_call_median_cold": round(us_cold, 1),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Gaussian random field, seeded N(0, s^2) weights)",
        "config": {"workload": f"fused 2D spectral block x[{B},{C},{H},{W}] n_modes{tuple(nm)} "
                               f"-> {m1}x{m2h} modes, linear skip, bias, erf GELU",
                   "batch": B, "channels": C, "H": H, "W": W, "modes": [m1, m2h],
                   "fused_path": bool(fused), "algorithmic_bytes": total_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved_block, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved_block / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(args.workload),
                     "us_per_call": round(us_events, 1),
                     "kernel": "fno_spectral_block_f32 (all launches of one call) on one stream; "
                               "HIP events on that stream around the timed steps, per call"},
        "copy_bandwidth_gbs": round(copy_gbs, 1),
        "torch_rocm_baseline": rocm,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(B, C, H, W, nm, total_bytes)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
