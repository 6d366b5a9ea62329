#!/usr/bin/env python3
"""Benchmark of the MI355X selective-scan hot path.

One "step" = one selective_scan forward (saving the chunk states) + one
backward at the Mamba-370M shape (batch 8, d_inner 2048,
d_state 16, L 2048; bf16 u/delta/z/B/C/dout, fp32 A/D/delta_bias, fp32
arithmetic), inputs resident in HBM.  Prints ONE JSON line:

  value     = algorithmic bytes of fwd+bwd (743,882,752 B) / time per step, GB/s
  roofline  = the dominant kernel (scan_bwd): its algorithmic bytes per launch /
              its average duration from HIP events on its launch stream
  cpu_baseline = the CPU oracle (fp32 torch, host threads) on a bounded sample
              of the same workload, in equivalent GB/s

plus the decode step (config 2, cold = Infinity Cache flushed between steps,
and warm), config 0 forward, config 3 forward+backward and config 4 end to end
(48-layer causal LM: prefill and greedy-decode tokens/s, share of time in the
scan / update kernels; also alone with --e2e).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# fp32 VALU issue ceiling of the MI355X: 256 CUs x 4 SIMDs x 16 lanes per
# clock at the 2.4 GHz peak engine clock, in lane-operations per second
# (packed fp32 forms are not used by this build)
VALU_PEAK_LANE_OPS = 256 * 4 * 16 * 2.4e9

# Stored counter results for the config-1 scan kernels, from rocprofv3 runs of
# `bench.py --profile-run` (commands and tables in
# profiles/scan_decode_hbm_bytes.md and profiles/scan_sq_counters_config1.md);
# counters cannot be read inside the timed run, so these are re-measured
# after each kernel change and reported with their source.
#   traffic: FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0 KiB per dispatch, the factors
#            being what the same counters read for a 256 MiB device copy;
#   valu:    SQ_INSTS_VALU wave instructions per dispatch (x 64 lanes).
TRAFFIC_BYTES = {"scan_fwd": (2 * 104_920 + 262_144) * 1024,
                 "scan_bwd": (2 * 303_709 + 381_512) * 1024}
VALU_INSTS = {"scan_fwd": 6.2962e7, "scan_bwd": 1.6993e8}
COUNTERS_SOURCE = "profiles/scan_decode_hbm_bytes.md, profiles/scan_sq_counters_config1.md"


def inputs(batch, dim, seqlen, nstate, dtype, dev, seed, delta_shift=0.0):
    import math

    import torch
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(batch, dim, seqlen, generator=g)
    delta = torch.randn(batch, dim, seqlen, generator=g) + delta_shift
    z = torch.randn(batch, dim, seqlen, generator=g)
    B = torch.randn(batch, nstate, seqlen, generator=g)
    C = torch.randn(batch, nstate, seqlen, generator=g)
    A = -torch.arange(1, nstate + 1, dtype=torch.float32)[None].expand(dim, nstate).contiguous()
    dt = torch.exp(torch.rand(dim, generator=g) * (math.log(0.1) - math.log(1e-3))
                   + math.log(1e-3)).clamp(min=1e-4)
    bias = dt + torch.log(-torch.expm1(-dt))
    D = torch.ones(dim)
    dout = torch.randn(batch, dim, seqlen, generator=g)
    c = dict(u=u, delta=delta, z=z, B=B, C=C, dout=dout)
    out = {k: v.to(dtype).to(dev) for k, v in c.items()}
    out.update(A=A.to(dev), D=D.to(dev), bias=bias.to(dev))
    return out


def scan_bytes(batch, dim, seqlen, nstate, s_in, has_z=True):
    s_z = s_in if has_z else 0
    fwd = (batch * dim * seqlen * (3 * s_in + s_z) + batch * nstate * seqlen * 2 * s_in
           + dim * nstate * 4 + 2 * dim * 4 + batch * dim * nstate * 4)
    bwd = (batch * dim * seqlen * (5 * s_in + 2 * s_z) + batch * nstate * seqlen * 4 * s_in
           + 2 * dim * nstate * 4 + 4 * dim * 4 + batch * dim * nstate * 4)
    return fwd, bwd


def time_scan(ss, N, x, steps, warmup, fwd_only=False, clock_warmup_ms=0.0, info=None):
    """Returns (ms per step from events around the loop, {kernel: avg ms}).

    The steps are timed twice, back to back: first with events around the
    loop only (the ms per step returned), then again with the library's HIP
    events around every kernel launch, on the launch stream (the per-kernel
    times returned).  Those per-kernel events cost about 20 us per step of
    their own (a barrier packet and a timestamp around each launch), so the
    step time is not taken from the instrumented pass; its ms per step is
    written to info["ms_per_step_profiled"].

    clock_warmup_ms: before the `warmup` steps, run untimed steps back to
    back until that much wall time has passed.  The engine clock of an idle
    GPU takes about 40 ms of continuous work to reach its steady state (a
    per-step trace of the first 600 steps of a process: 2.6 ms/step over the
    first 5, 0.64 over steps 10-25, 0.56 from step 50 on; after 1 s idle the
    first 20 steps run 15% slow again), so a short --warmup alone times the
    ramp.  The steps it took are written to info["clock_warmup_steps"]."""
    import time

    import torch

    def step():
        # training step: the forward also keeps the ungated output for dz
        y = None if fwd_only else torch.empty_like(x["u"])
        out, h = ss.forward(x["u"], x["A"], x["B"], x["C"], x["D"], x["delta"], x["bias"],
                            None, None, None, z=x["z"], save_chunks=not fwd_only, out_ungated=y)
        if not fwd_only:
            ss.backward(x["u"], x["A"], x["B"], x["C"], x["D"], x["delta"], x["bias"], h, None,
                        x["dout"], None, z=x["z"], out_ungated=y)

    n_clock = 0
    if clock_warmup_ms > 0:
        t0 = time.perf_counter()
        while (time.perf_counter() - t0) * 1e3 < clock_warmup_ms:
            for _ in range(8):
                step()
            n_clock += 8
            torch.cuda.synchronize()
    if info is not None:
        info["clock_warmup_steps"] = n_clock
        info["clock_warmup_ms"] = clock_warmup_ms
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()

    def timed(profiled):
        if profiled:
            N.profile_begin()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        prof = N.profile_end() if profiled else {}
        return e0.elapsed_time(e1) / steps, prof

    ms, _ = timed(False)
    ms_prof, prof = timed(True)
    if info is not None:
        info["ms_per_step_profiled"] = ms_prof
    return ms, {k: v[1] / v[0] for k, v in prof.items()}


def time_decode(su, dev, steps, cold):
    """Config 2 decode loop: `steps` in-place decode steps captured in one HIP
    graph and replayed back to back (no host launch overhead), timed with
    events around the replay.  Cold: the steps rotate over 16 independent
    state tensors (336 MB > the 256 MB Infinity Cache), so every step streams
    its state from HBM; warm: every step updates the same state.  Returns
    microseconds per step."""
    import math

    import torch
    batch, dim, nstate = 64, 5120, 16
    g = torch.Generator().manual_seed(2)
    nbuf = 16 if cold else 1
    states = [(torch.randn(batch, dim, nstate, generator=g) * 0.1).to(dev) for _ in range(nbuf)]
    A = -torch.arange(1, nstate + 1, dtype=torch.float32)[None].expand(dim, nstate).contiguous().to(dev)
    dt0 = torch.exp(torch.rand(dim, generator=g) * (math.log(0.1) - math.log(1e-3))
                    + math.log(1e-3)).clamp(min=1e-4)
    bias = (dt0 + torch.log(-torch.expm1(-dt0))).to(dev)
    D = torch.ones(dim, device=dev)
    xs = [(torch.randn(batch, dim, generator=g).bfloat16().to(dev),
           torch.randn(batch, dim, generator=g).bfloat16().to(dev),
           torch.randn(batch, dim, generator=g).bfloat16().to(dev),
           torch.randn(batch, nstate, generator=g).bfloat16().to(dev),
           torch.randn(batch, nstate, generator=g).bfloat16().to(dev)) for _ in range(8)]
    out = torch.empty(batch, dim, dtype=torch.bfloat16, device=dev)

    def one(k):
        x, dt, z, B, C = xs[k % len(xs)]
        su.apply_ext(x, A, B, C, D, dt, bias, states[k % nbuf], z=z, inplace=True, out=out)

    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for k in range(4):
            one(k)
    torch.cuda.current_stream(dev).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for k in range(steps):
            one(k)
    graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return 1e3 * e0.elapsed_time(e1) / steps


def time_decode_flush(su, dev, steps, flush_mb=512):
    """Config 2 decode steps with the Infinity Cache flushed before each one:
    a `flush_mb` MB fill kernel between consecutive steps, all captured in
    one HIP graph; a second graph holds the fills alone, and the difference
    of the two replays is the time of the steps.  Returns microseconds per
    step."""
    import math

    import torch
    batch, dim, nstate = 64, 5120, 16
    g = torch.Generator().manual_seed(2)
    state = (torch.randn(batch, dim, nstate, generator=g) * 0.1).to(dev)
    A = -torch.arange(1, nstate + 1, dtype=torch.float32)[None].expand(dim, nstate).contiguous().to(dev)
    dt0 = torch.exp(torch.rand(dim, generator=g) * (math.log(0.1) - math.log(1e-3))
                    + math.log(1e-3)).clamp(min=1e-4)
    bias = (dt0 + torch.log(-torch.expm1(-dt0))).to(dev)
    D = torch.ones(dim, device=dev)
    x, dt, z = (torch.randn(batch, dim, generator=g).bfloat16().to(dev) for _ in range(3))
    B, C = (torch.randn(batch, nstate, generator=g).bfloat16().to(dev) for _ in range(2))
    out = torch.empty(batch, dim, dtype=torch.bfloat16, device=dev)
    return time_after_flush(
        dev, lambda: su.apply_ext(x, A, B, C, D, dt, bias, state, z=z, inplace=True, out=out),
        steps, flush_mb)


def time_copy_flush(dev, nbytes, steps, flush_mb=512):
    """A plain device-to-device copy of `nbytes` (torch's copy kernel) timed
    as time_decode_flush times the decode step: the reference for what a
    kernel that reads and writes that many bytes costs from a flushed cache.
    Returns microseconds per copy."""
    import torch
    src = torch.randn(nbytes // 4, device=dev)
    dst = torch.empty_like(src)
    return time_after_flush(dev, lambda: dst.copy_(src), steps, flush_mb)


def time_after_flush(dev, fn, steps, flush_mb):
    """`steps` calls of fn, each after a `flush_mb` MB fill kernel, captured
    in one HIP graph; a second graph holds the fills alone, and the difference
    of the two replays is the time of the calls.  Returns microseconds per
    call."""
    import torch
    # float32, so the fill is a kernel (a byte pattern could become a memset node)
    junk = torch.empty((flush_mb << 20) // 4, dtype=torch.float32, device=dev)

    def run(with_steps):
        for k in range(steps):
            junk.fill_(float(k))
            if with_steps:
                fn()

    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        run(True)
    torch.cuda.current_stream(dev).wait_stream(side)
    times = []
    for with_steps in (True, False):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run(with_steps)
        graph.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
        del graph
    del junk
    return 1e3 * (times[0] - times[1]) / steps


def time_host_overhead(dev, calls=200):
    """Per-call cost of the operator API on the host next to the kernel time:
    SelectiveUpdateFn.apply at config 2 (B=64, D=5120, N=16, bf16 vectors,
    fp32 state) and SelectiveScanFn.apply (forward, inference) at batch 4,
    2048 channels, L=2048, N=16 (the config-4 prefill shape).  host_us: time
    to enqueue one call (Python, argument checks, allocation, launch);
    wall_us: per call over a loop ended by a synchronize; kernel_us: the
    library's kernel time from HIP events."""
    import math

    import torch

    from ssm_mamba_amd import _native as N
    from ssm_mamba_amd.ops import SelectiveScanFn, SelectiveUpdateFn
    res = {}
    g = torch.Generator().manual_seed(3)
    b, d, n = 64, 5120, 16
    st = (torch.randn(b, d, n, generator=g) * 0.1).to(dev)
    A = -torch.arange(1, n + 1, dtype=torch.float32)[None].expand(d, n).contiguous().to(dev)
    dt0 = torch.exp(torch.rand(d, generator=g) * (math.log(0.1) - math.log(1e-3))
                    + math.log(1e-3)).clamp(min=1e-4)
    bias = (dt0 + torch.log(-torch.expm1(-dt0))).to(dev)
    D = torch.ones(d, device=dev)
    u, dt = (torch.randn(b, d, generator=g).bfloat16().to(dev) for _ in range(2))
    B, C = (torch.randn(b, n, generator=g).bfloat16().to(dev) for _ in range(2))
    cases = {"SelectiveUpdateFn.apply config2":
             lambda: SelectiveUpdateFn.apply(u, A, B, C, D, dt, bias, st)}
    bs, ds, L = 4, 2048, 2048
    us = torch.randn(bs, ds, L, generator=g).bfloat16().to(dev)
    dls = torch.randn(bs, ds, L, generator=g).bfloat16().to(dev)
    Bs, Cs = (torch.randn(bs, n, L, generator=g).bfloat16().to(dev) for _ in range(2))
    As = A[:ds].contiguous()
    cases["SelectiveScanFn.apply fwd B4 D2048 L2048"] = \
        lambda: SelectiveScanFn.apply(us, As, Bs, Cs, D[:ds], dls, bias[:ds])
    with torch.no_grad():
        for name, fn in cases.items():
            for _ in range(10):
                fn()
            torch.cuda.synchronize()
            N.profile_begin()
            t0 = time.perf_counter()
            for _ in range(calls):
                fn()
            t1 = time.perf_counter()
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            prof = N.profile_end()
            kern = sum(v[1] for v in prof.values()) / calls
            res[name] = {"host_us": round(1e6 * (t1 - t0) / calls, 2),
                         "wall_us": round(1e6 * (t2 - t0) / calls, 2),
                         "kernel_us": round(1e3 * kern, 2)}
    return res


def decode_eager(su, dev, steps):
    """Config 2 decode steps launched one by one over 16 rotating states (for
    counter runs, which see each launch as its own dispatch)."""
    import torch
    batch, dim, nstate = 64, 5120, 16
    g = torch.Generator().manual_seed(2)
    states = [(torch.randn(batch, dim, nstate, generator=g) * 0.1).to(dev) for _ in range(16)]
    A = -torch.arange(1, nstate + 1, dtype=torch.float32)[None].expand(dim, nstate).contiguous().to(dev)
    bias = torch.full((dim,), -4.0, device=dev)
    D = torch.ones(dim, device=dev)
    x, dt, z = (torch.randn(batch, dim, generator=g).bfloat16().to(dev) for _ in range(3))
    B, C = (torch.randn(batch, nstate, generator=g).bfloat16().to(dev) for _ in range(2))
    out = torch.empty(batch, dim, dtype=torch.bfloat16, device=dev)
    for k in range(steps):
        su.apply_ext(x, A, B, C, D, dt, bias, states[k % 16], z=z, inplace=True, out=out)


def time_e2e(dev, decode_steps: int = 128, reps: int = 3):
    """Config 4, end to end: the causal LM of ssm_mamba_amd.causal_lm at 48
    layers, d_model 1024 (d_inner 2048, N 16, conv 4, dt_rank 64), vocab 50280,
    bf16 weights with random init, eval mode.  Prefill = generate's prefill over
    4 x 2048 random token ids (id 0 is the pad id, so rows may be shorter and
    take the left-padding length path): every layer over the prompt, caching
    the decode state, and the final norm and LM head at position lengths - 1
    of each row (the full-logits forward is reported beside it); decode = exactly
    `decode_steps` greedy steps (48 layers + norm + LM head + pick each), the
    step captured once in a HIP graph and replayed.  Returns tokens/s for both
    and the share of time in the scan / state-update kernels: for the prefill
    from the library's per-kernel HIP events (forward scan, its segment
    summaries and the B/C prep); for the decode, the 48 layers run as one
    kernel (ssm_decode_layers, whose state update cannot be timed apart), so
    the step reports that kernel's share from a graph of it alone, and for
    reference a graph of 48 stand-alone state-update kernels on the same
    buffers."""
    import torch

    from ssm_mamba_amd import _native as N
    from ssm_mamba_amd import decode as DEC
    from ssm_mamba_amd import selective_update as su
    from ssm_mamba_amd.causal_lm import CausalLM, CausalLMConfig

    torch.manual_seed(4)
    cfg = CausalLMConfig(vocab_size=50280, model_dim=1024, state_dim=16, num_layers=48,
                         device=str(dev))
    model = CausalLM(cfg).to(dev, torch.bfloat16).eval()
    n_params = sum(p.numel() for p in model.parameters())
    batch, seqlen = 4, 2048
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, cfg.vocab_size, (batch, seqlen), generator=g).to(dev)
    lengths = (ids != cfg.pad_token_id).sum(dim=1)
    ev = lambda: torch.cuda.Event(enable_timing=True)
    dec = model.decoder(batch, decode_steps + 1)
    with torch.no_grad():
        dec.capture()
        dec.prefill(ids, lengths)
        dec.replay(2)
        torch.cuda.synchronize()
        def median_ms(fn):
            times = []
            for _ in range(reps):
                e0, e1 = ev(), ev()
                e0.record()
                fn()
                e1.record()
                torch.cuda.synchronize()
                times.append(e0.elapsed_time(e1))
            return sorted(times)[len(times) // 2]

        # generate's prefill: the LM head only at each row's last position
        pre_ms = median_ms(lambda: model.forward_last(ids, lengths, use_cache=True))
        # forward with the logits of every position, for reference
        full_ms = median_ms(lambda: model(ids, lengths, use_cache=True))
        N.profile_begin()
        model.forward_last(ids, lengths, use_cache=True)
        prof = N.profile_end()
        scan_ms = sum(v[1] for k, v in prof.items() if k in ("scan_fwd", "scan_fwd_segsum", "bc_prep"))

        dec.prefill(ids, lengths)
        torch.cuda.synchronize()
        e0, e1 = ev(), ev()
        e0.record()
        dec.replay(decode_steps)
        e1.record()
        torch.cuda.synchronize()
        dec_ms = e0.elapsed_time(e1)
        new_tokens = dec.tokens[:, :decode_steps + 1].clone()

        # the step's 48 state-update kernels alone (the fused decode kernel that
        # also applies the dt projection and the gate), on the model's buffers
        inner, nstate = 2 * cfg.model_dim, cfg.state_dim
        layers = [l.ssm for l in model.layers]
        rank = layers[0].delta_rank
        params = torch.randn(batch, rank + 2 * nstate, device=dev).bfloat16()
        nparts = DEC.xproj_blocks(inner, rank + 2 * nstate) if DEC.FOLD_XPROJ else 0
        # with the x-projection folded, the kernel also adds its partials
        parts = (torch.randn(nparts, batch, (rank + 2 * nstate + 3) // 4 * 4, device=dev) / nparts
                 if nparts else None)
        xc = torch.randn(batch, inner, device=dev).bfloat16()
        xz = torch.randn(batch, 2 * inner, device=dev).bfloat16()
        fused = DEC.block_step_supported(layers[0], torch.zeros(batch, cfg.model_dim, device=dev,
                                                                dtype=torch.bfloat16),
                                         model.layers[0].norm.weight)

        def updates():
            for m in layers:
                if fused:
                    DEC.ssm_step(params if parts is None else parts, rank, m.delta_proj.weight,
                                 m.delta_proj.bias, m.log_A, m.D, xc, xz, m._ssm_hiddens)
                else:
                    su.apply_ext(xc, -torch.exp(m.log_A.float()), params[:, :nstate].contiguous(),
                                 params[:, :nstate].contiguous(), m.D.float(), xc,
                                 m.delta_proj.bias.float(), m._ssm_hiddens, z=xc, inplace=True)

        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            updates()
        torch.cuda.current_stream(dev).wait_stream(side)
        ug = torch.cuda.CUDAGraph()
        with torch.cuda.graph(ug):
            updates()
        ug.replay()
        torch.cuda.synchronize()
        e0, e1 = ev(), ev()
        e0.record()
        for _ in range(decode_steps):
            ug.replay()
        e1.record()
        torch.cuda.synchronize()
        upd_ms = e0.elapsed_time(e1)

        # the step's layer chain alone (one launch for the 48 layers)
        x0 = torch.randn(batch, cfg.model_dim, device=dev).bfloat16()
        chain = DEC.layers_supported(model.layers, x0)
        chain_ms = 0.0
        if chain:
            with torch.cuda.stream(side):
                DEC.layers_step(model, model.layers, x0)
            torch.cuda.current_stream(dev).wait_stream(side)
            cg = torch.cuda.CUDAGraph()
            with torch.cuda.graph(cg):
                DEC.layers_step(model, model.layers, x0)
            cg.replay()
            torch.cuda.synchronize()
            e0, e1 = ev(), ev()
            e0.record()
            for _ in range(decode_steps):
                cg.replay()
            e1.record()
            torch.cuda.synchronize()
            chain_ms = e0.elapsed_time(e1)
            DEC.layers_check(model)
    res = {
        "config": "48 layers, d_model 1024, d_inner 2048, N 16, d_conv 4, dt_rank 64, vocab 50280, "
                  "bf16 weights (random init), eval; prefill 4 x 2048 (pad id 0 -> lengths), then "
                  f"{decode_steps} greedy steps replayed from one HIP graph",
        "params": n_params,
        "prompt_lengths": lengths.tolist(),
        "prefill_ms": round(pre_ms, 3),
        "prefill_note": "generate's prefill: the LM head at each row's position lengths - 1 only",
        "prefill_all_logits_ms": round(full_ms, 3),
        "prefill_tokens_per_s": round(batch * seqlen / (pre_ms * 1e-3), 1),
        "prefill_scan_share": round(scan_ms / pre_ms, 4),
        "prefill_scan_ms": round(scan_ms, 3),
        "decode_ms_per_step": round(dec_ms / decode_steps, 4),
        "decode_tokens_per_s": round(batch * decode_steps / (dec_ms * 1e-3), 1),
        "decode_layer_chain": bool(chain),
        "decode_layer_chain_share": round(chain_ms / dec_ms, 4),
        "decode_layer_chain_us_per_step": round(1e3 * chain_ms / decode_steps, 2),
        "decode_standalone_update_us_per_step": round(1e3 * upd_ms / decode_steps, 2),
        "decode_fused_kernels": bool(fused),
        "first_new_tokens": new_tokens[0, :8].tolist(),
    }
    del model, dec
    torch.cuda.empty_cache()
    return res


def cpu_baseline(seconds: float):
    """Times the CPU oracle (fp32 torch) forward+backward on the config-1 shape
    with a reduced channel count, sized to run about `seconds`."""
    import torch

    from oracle import scan_ref as R
    cpus = os.cpu_count() or 1
    usable = _usable_cpus()
    threads = min(cpus, usable)
    torch.set_num_threads(threads)

    def run(dim):
        c = R.make_inputs(8, dim, 2048, 16, seed=0, dtype=torch.bfloat16, with_z=True)
        dy = torch.randn(8, dim, 2048, generator=torch.Generator().manual_seed(1)).bfloat16()
        t = time.perf_counter()
        R.scan_fwd(c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["delta_bias"], z=c["z"],
                   chunk=None, dtype=torch.float32)
        R.scan_bwd(c["u"], c["delta"], c["A"], c["B"], c["C"], c["D"], c["delta_bias"], z=c["z"],
                   dy=dy, dtype=torch.float32)
        return time.perf_counter() - t

    # calibrate on 256 channels (large enough for per-op overhead not to
    # dominate), then size the timed sample to about `seconds`
    dim, t = 256, run(256)
    target = int(min(2048, 256 * seconds / max(t, 1e-3)) // 256 * 256)
    if target > dim:
        dim, t = target, run(target)
    tok_ch = 8 * dim * 2048
    fwd, bwd = scan_bytes(8, 2048, 2048, 16, 2)
    per_tc = (fwd + bwd) / (8 * 2048 * 2048)
    return {
        "value": round(tok_ch / t * per_tc / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle/scan_ref.py fp32 fwd+bwd, batch 8 x {dim} channels x L 2048 x N 16 "
                   f"with z ({t:.1f} s); GB/s = token-channels/s x config-1 bytes per "
                   f"token-channel ({per_tc:.2f})"),
        "tokens_channels_per_s": round(tok_ch / t, 1),
        "cpu_model": _cpu_model(),
        "cpu_count": cpus,
        "cpus_usable": usable,
        "threads_note": ("torch.set_num_threads(os.cpu_count()) as planned, capped at the "
                         "CPUs this process may run on (affinity and cgroup quota)"),
    }


def _usable_cpus() -> int:
    """CPUs this process can run on at once: its affinity set, capped by the
    cgroup CPU quota when one is set."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            n = min(n, max(1, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return max(1, n)


def _cpu_model() -> str:
    """The CPU model name as lscpu prints it (falls back to /proc/cpuinfo)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.strip().startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_config3(ss, N, dev, steps=10, warmup=2):
    """B=1, D=2560, L=16384, N=16, fp32, z, delta_raw
    shifted by +2; the sequence split (40 channel blocks fill 40 of 256 CUs).
    summary_share: the two segment-summary kernels' part of the kernel time."""
    import torch
    x3 = inputs(1, 2560, 16384, 16, torch.float32, dev, seed=3, delta_shift=2.0)
    ms3, k3 = time_scan(ss, N, x3, steps, warmup, clock_warmup_ms=50.0)
    f3, b3 = scan_bytes(1, 2560, 16384, 16, 4)
    summ = k3.get("scan_fwd_segsum", 0.0) + k3.get("scan_bwd_segsum", 0.0)
    return {"ms_per_step": round(ms3, 4), "GBs": round((f3 + b3) / (ms3 * 1e-3) / 1e9, 1),
            "kernels_ms": {k: round(v, 4) for k, v in k3.items()},
            "summary_share": round(summ / sum(k3.values()), 4)}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    # the engine clock takes about 40 ms of continuous work to settle (see
    # time_scan); this untimed warm-up runs ahead of --warmup and is reported
    # in the JSON line as "clock_warmup"
    ap.add_argument("--clock-warmup-ms", type=float, default=200.0,
                    help="untimed config-1 steps run back to back for this long before --warmup")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-extra", action="store_true", help="only the config-1 step")
    ap.add_argument("--no-e2e", action="store_true", help="skip config 4 (end to end)")
    ap.add_argument("--e2e", action="store_true",
                    help="only config 4 end to end (causal LM prefill + 128 decode steps); "
                         "prints its own JSON line")
    ap.add_argument("--config3", action="store_true",
                    help="only config 3 (B=1, D=2560, L=16384, fp32, sequence split) fwd+bwd; "
                         "prints its own JSON line (for a kernel trace of that config)")
    ap.add_argument("--profile-run", action="store_true",
                    help="for rocprofv3 counter runs: one 256 MiB device-to-device copy (reference for "
                         "the byte counters), config-1 fwd+bwd (--steps times), 32 eager config-2 "
                         "decode steps; no JSON")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (--gpus 1); the multi-GPU "
              "sharding of the scan is a design, not a measured path", file=sys.stderr)
        sys.exit(2)

    import torch

    from ssm_mamba_amd import _native as N
    from ssm_mamba_amd import selective_scan as ss
    from ssm_mamba_amd import selective_update as su

    dev = torch.device("cuda:0")
    N.lib()
    batch, dim, seqlen, nstate = 8, 2048, 2048, 16
    x = inputs(batch, dim, seqlen, nstate, torch.bfloat16, dev, seed=1)
    if args.e2e:
        print(json.dumps({"e2e": time_e2e(dev)}), flush=True)
        return
    if args.config3:
        print(json.dumps({"config3_fwd_bwd": time_config3(ss, N, dev)}), flush=True)
        return
    if args.profile_run:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)  # 256 MiB read + 256 MiB written
        del src, dst
        time_scan(ss, N, x, args.steps, args.warmup)
        decode_eager(su, dev, 32)
        torch.cuda.synchronize()
        print("profile run done", flush=True)
        return
    fwd_b, bwd_b = scan_bytes(batch, dim, seqlen, nstate, 2)
    cw = {}
    ms, kern = time_scan(ss, N, x, args.steps, args.warmup, clock_warmup_ms=args.clock_warmup_ms,
                         info=cw)
    gbs = (fwd_b + bwd_b) / (ms * 1e-3) / 1e9
    t_fwd, t_bwd = kern.get("scan_fwd", 0.0), kern.get("scan_bwd", 0.0)
    if t_bwd >= t_fwd:
        dom, dom_bytes, dom_ms = "scan_bwd", bwd_b, t_bwd
    else:
        dom, dom_bytes, dom_ms = "scan_fwd", fwd_b, t_fwd
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    valu = VALU_INSTS[dom] * 64 / (dom_ms * 1e-3)
    res = {
        "metric": "scan fwd+bwd GB/s (% HBM peak) at 370M shape; state-update us/decode step",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_warmup": {"steps": cw["clock_warmup_steps"], "ms": cw["clock_warmup_ms"],
                         "note": "untimed steps run back to back ahead of --warmup until the "
                                 "engine clock settles (about 40 ms of work from idle)"},
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "io_dtype": "bf16",
        "data": "synthetic (seeded; reference init distributions)",
        "config": {"workload": "selective_scan forward+backward, Mamba-370M shape (BASELINE config 1)",
                   "batch": batch, "d_inner": dim, "d_state": nstate, "seqlen": seqlen,
                   "z_gate": True, "parallelism": "single GPU"},
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "tokens_channels_per_s": round(batch * dim * seqlen / (ms * 1e-3), 1),
        "kernels_ms": {k: round(v, 4) for k, v in kern.items()},
        "kernels_note": "HIP events around each launch, on its stream, over a second pass of the "
                        "same timed steps; those events add about 20 us per step "
                        f"({cw['ms_per_step_profiled']:.4f} ms per step with them), so ms_per_step "
                        "and value come from the pass without them",
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": TRAFFIC_BYTES.get(dom), "traffic_unit": "B",
                     "traffic_source": "stored counter run: " + COUNTERS_SOURCE,
                     "algorithmic_bytes_per_launch": dom_bytes, "avg_launch_ms": round(dom_ms, 4)},
        # the ceiling the scan kernels actually meet: VALU instruction issue
        "roofline_valu": {"kernel": dom, "bound": "valu",
                          "achieved": round(valu / 1e12, 3), "peak": round(VALU_PEAK_LANE_OPS / 1e12, 3),
                          "unit": "T lane-ops/s", "frac": round(valu / VALU_PEAK_LANE_OPS, 4),
                          "valu_insts_per_launch": VALU_INSTS[dom],
                          "source": "SQ_INSTS_VALU x 64 from " + COUNTERS_SOURCE},
    }
    if not args.no_extra:
        floor_us = 44_937_216 / (HBM_PEAK_GBS * 1e3)
        cold = time_decode(su, dev, 256, cold=True)
        warm = time_decode(su, dev, 256, cold=False)
        flushed = time_decode_flush(su, dev, 256)
        copy_us = time_copy_flush(dev, 64 * 5120 * 16 * 4, 256)
        res["decode"] = {"config": "B=64 D=5120 N=16, fp32 state, bf16 x/dt/z/B/C, 256 steps "
                                   "replayed from one HIP graph; cold: a 512 MB fill between "
                                   "steps (flush), and 16 rotating states (rotation)",
                         "us_per_step_cold": round(flushed, 3),
                         "us_per_step_cold_rotation": round(cold, 3),
                         "us_per_step_warm": round(warm, 3),
                         "floor_us": round(floor_us, 3),
                         "cold_over_floor": round(flushed / floor_us, 3),
                         "cold_GBs": round(44_937_216 / (flushed * 1e-6) / 1e9, 1),
                         # torch's device copy of the state's 21 MB (42 MB moved against
                         # the step's 45 MB), timed the same way
                         "copy_state_bytes_us_cold": round(copy_us, 3),
                         "cold_over_copy": round(flushed / copy_us, 3)}
        res["host_overhead"] = time_host_overhead(dev)
        x0 = inputs(2, 1536, 512, 16, torch.float32, dev, seed=0)
        ms0, k0 = time_scan(ss, N, x0, 20, 3, fwd_only=True, clock_warmup_ms=50.0)
        f0, _ = scan_bytes(2, 1536, 512, 16, 4)
        # ms: the whole forward call (its segment summaries and scan, events
        # around the loop); kernels_ms: each kernel from the instrumented pass
        res["config0_fwd"] = {"ms": round(ms0, 4), "GBs": round(f0 / (ms0 * 1e-3) / 1e9, 1),
                              "kernels_ms": {k: round(v, 4) for k, v in k0.items()}}
        del x0
        res["config3_fwd_bwd"] = time_config3(ss, N, dev)
        try:
            if not args.no_e2e:
                res["e2e"] = time_e2e(dev)
        except Exception as exc:  # reported, not fatal to the headline line
            res["e2e"] = {"error": f"{type(exc).__name__}: {exc}"}
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
