#!/usr/bin/env python3
"""Benchmark: drinkme's fused radix decode + GEMV on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Workloads (seeded synthetic weights, drinkme_amd/synth.py):
  qwen3-8b-step   (default) one Qwen3-8B decode step's compressed Linears:
                  36 layers x q/k/v/o/gate/up/down + lm_head = 253 GEMVs,
                  N(0, 0.02) weights packed at sip, M = 1, bf16 x ~ N(0, 1)
  qwen3-8b-layer  one such layer (7 GEMVs), four copies rotated
  32b-layer       one layer of the 32B-class stack (hidden 5120: q 8192 x 5120,
                  k/v 1024 x 5120, o 5120 x 8192, gate/up 25600 x 5120, down
                  5120 x 25600), Student-t(4) weights scaled to std 0.02, two
                  copies rotated
  linear-4096     one 4096 x 4096 tensor (rotated over 32 packed copies so
                  the 256 MB last-level cache cannot hold them)
--profile sip | gulp | balanced packs the weights at that profile; --m sets
the activation rows (1 = decode, 4 = the MTP verify rows).

A step is one sweep over the workload's GEMVs, captured once as a HIP graph
and replayed; inputs are resident in HBM before timing starts. The GEMVs
that share an activation in a decoder layer (q/k/v; gate/up) run as one
grouped launch (dmx_radix_gemv_group), the others one launch each. Also
timed: the same sweep with one launch per GEMV (config.ungrouped), and
without a graph, the way a serving loop calls it: one radix_ops call per
Linear (config.eager_ungrouped), and one module call per Linear with the
q/k/v and gate/up modules in shared-input groups (config.eager_modules).
For gulp at M = 3..4 the sweep is also timed with its verify rows on the
matrix cores (radix_ops.set_policy("matrix"), config.matrix_cores). The
ceiling beside it (config.read_wall): the same launches as plain
non-temporal reads of their bytes (dmx_read_probe), in a graph timed the
same way, the largest launch's bytes read alone, and per launch kind (each
kind's launches in a graph of their own) the kernel against the read.
Reported:
  value       whole-sweep compressed-HBM GB/s = sum of algorithmic bytes /
              step time, B = 4 NW + 4 (R NB + 1) + P + 2 M C + 2 M R per
              GEMV (payload, directory, palette P = 7 sip / 21 gulp, bf16 x
              and out; not the pad)
  roofline    the dominant kernel launch (the grouped gate/up GEMV of a
              layer, 2 x 12288 x 4096): its algorithmic bytes per launch /
              its average launch time, from HIP events around a graph of
              its launches, timed after 0.3 s of untimed replays (the
              first thing timed: the clocks settle first)
  cpu_baseline  drinkme's CPU route on the host's cores: the compiled
              drinkme decoder (oracle/_ref) + torch F.linear, on a bounded
              sample (layer 0), scaled to the step by weight count; three
              legs (every thread of the job's CPU share, one thread, and
              F.linear over the cached decoded weight), `value` the first;
              nproc and the CPUs the process may run on are recorded
One JSON line goes to stdout; progress lines go to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_GBPS = 8000.0  # MI355X HBM3E
PALETTE_BYTES = {"sip": 7, "balanced": 10, "gulp": 21}
CPU_SHARE = 16  # host threads the CPU legs use at most: one GPU's share of its host's cores


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic_bytes(rt: dict, m: int = 1) -> int:
    R, C = int(rt["R"]), int(rt["C"])
    nb = -(-C // int(rt["block_size"]))
    return 4 * int(rt["NW"]) + 4 * (R * nb + 1) + PALETTE_BYTES[rt["profile"]] + 2 * m * C + 2 * m * R


def workload_items(name: str):
    """(workload, layer, tensor, rows, cols, distribution) per GEMV."""
    from drinkme_amd import synth

    N, T4 = synth.NORMAL, synth.STUDENT_T4
    if name == "qwen3-8b-step":
        return [("qwen3-8b", layer, n, r, c, N) for layer, n, r, c in synth.qwen3_8b_step()]
    if name == "qwen3-8b-layer":
        # four copies of the layer, so the sweep is not held by the 256 MB cache
        return [("qwen3-8b", copy, n, r, c, N) for copy in range(4) for n, r, c in synth.QWEN3_8B_LAYER]
    if name == "32b-layer":
        return [("32b-class", copy, n, r, c, T4) for copy in range(2) for n, r, c in synth.CLASS_32B_LAYER]
    if name == "linear-4096":
        return [("linear-4096", copy, "w", 4096, 4096, N) for copy in range(32)]
    raise SystemExit(f"unknown workload {name!r}")


def build_tensors(items, profile: str, m: int = 1):
    import numpy as np  # noqa: F401

    from drinkme_amd import radix_pack, swap, synth

    tensors = []
    t0 = time.time()
    last = t0
    for i, (wl, layer, name, R, C, dist) in enumerate(items):
        bits = synth.weight(wl, layer, name, R, C, dist)
        p = radix_pack.pack_array_radix(bits, profile)
        if p is None:
            raise SystemExit(f"{wl}/{layer}/{name}: radix would expand this tensor")
        rt = swap.to_device_radix(p, "cuda")
        tensors.append({"layer": layer, "name": name, "R": R, "C": C, "rt": rt, "bytes": algorithmic_bytes(rt, m),
                        "bf16_bytes": 2 * R * C, "bpw": p["bpw"]})
        if time.time() - last > 10 or i + 1 == len(items):
            last = time.time()
            log(f"packed {i + 1}/{len(items)} tensors ({last - t0:.0f} s)")
    return tensors


def time_graph(fn, replays: int, warmup: int, settle_s: float = 0.0, info: dict | None = None) -> float:
    """Milliseconds per replay of `fn` captured as a HIP graph. settle_s:
    untimed replays for at least that long before the warmup ones (the GPU
    comes out of the host-side packing at low clocks: a graph timed first,
    over a few ms, reads up to 12% slow); their count goes to info."""
    import torch

    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    settle, t0 = 0, time.time()
    while time.time() - t0 < settle_s:
        for _ in range(10):
            g.replay()
        settle += 10
        torch.cuda.synchronize()
    if info is not None:
        info["settle_replays"] = settle
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / replays


def time_eager(fn, reps: int, warmup: int) -> tuple:
    """(milliseconds per call of `fn` on the GPU's clock, milliseconds the
    host spent issuing one call): `fn` launched eagerly, no graph, HIP
    events around `reps` calls after `warmup` untimed ones."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    host_ms = (time.perf_counter() - t0) * 1e3 / reps
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps, host_ms


def cpu_baseline(tensors, xs, budget_s: float = 10.0):
    """drinkme's CPU route (src/drinkme/codec/swap.py:344-352): decode the
    weight with drinkme's compiled C++ decoder (oracle/_ref; the oracle's C
    decoder when that library is absent), then torch F.linear on the bf16
    weight. Three legs, each on a bounded sample of the workload and scaled
    to the whole sweep by weight count:
      cpu_share   decode on every thread of the job's CPU share (the CPUs
                  the process may run on, at most 16: a one-GPU job's share
                  of its host) over row ranges + F.linear on as many; per
                  call (value is this leg's rate)
      one_thread  decode and F.linear on one thread: the serve route's own
                  decode runs single-threaded (radix_native.py:221, called
                  without workers from radix_pack.py:292-294)
      cached_w    F.linear alone over the already-decoded weight, every
                  thread: the CPU route after its first call, which keeps
                  the decoded weight (swap.py:350-351)"""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    import torch

    from oracle import radix_oracle as O

    kind = "reference" if O.ref_available() else "port"
    nproc = os.cpu_count() or 1
    allowed = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    threads = max(1, min(allowed, CPU_SHARE))
    sample = [t for t in tensors if t["layer"] == tensors[0]["layer"]]
    host = []
    for t in sample:
        rt = t["rt"]
        host.append((rt["rx_palette_np"], rt["rx_offsets"].cpu().numpy(),
                     rt["rx_data"][: rt["NW"]].cpu().numpy(), t["R"], t["C"], tuple(rt["widths"])))
    xcpu = {c: x.cpu() for c, x in xs.items()}
    total_w = sum(t["R"] * t["C"] for t in tensors)
    total_bytes = sum(t["bytes"] for t in tensors)

    def decode(h, nthreads):
        pal, off, data, R, C, widths = h
        out = np.empty((R, C), np.uint16)
        step = -(-R // (4 * nthreads)) if nthreads > 1 else R
        if kind == "reference":
            job = lambda r: O.ref_decode(pal, off, data, R, C, widths, r, min(step, R - r), out[r:])  # noqa: E731
        else:
            pk = O.Pack((R, C), 1024, widths, pal, off, data)
            job = lambda r: O.decode_rows(pk, r, min(step, R - r), out[r:])  # noqa: E731
        if nthreads > 1:
            with ThreadPoolExecutor(nthreads) as ex:
                list(ex.map(job, range(0, R, step)))
        else:
            job(0)
        return torch.from_numpy(out.view(np.int16)).view(torch.bfloat16)

    def timed(fn, items, budget, max_reps=20):
        """Seconds per pass over `items` (whole passes within the budget, at
        least one), and the passes made. A pass stops early when one item
        alone exceeds the budget: then the weights it covered are returned."""
        reps, t0, covered = 0, time.time(), 0
        while True:
            covered = 0
            for h in items:
                fn(h)
                covered += h[3] * h[4]
                if reps == 0 and time.time() - t0 > budget:
                    break
            reps += 1
            if time.time() - t0 > budget or reps >= max_reps:
                break
        return (time.time() - t0) / reps, reps, covered

    def leg(name, per_pass_s, weights, reps, cores, what):
        step_s = per_pass_s * total_w / weights
        return {"value": total_bytes / step_s / 1e9, "unit": "GB/s", "cores": cores, "ms_per_step": step_s * 1e3,
                "sample": f"{what}: {weights / 1e6:.1f} M weights of layer {sample[0]['layer']} x{reps}, "
                          f"scaled by weight count to the sweep ({total_w / 1e9:.3f} G weights)"}

    legs = {}
    torch.set_num_threads(threads)
    per, reps, w = timed(lambda h: torch.nn.functional.linear(xcpu[h[4]], decode(h, threads)), host, budget_s)
    legs["cpu_share"] = leg("cpu_share", per, w, reps, threads,
                            f"decode (drinkme C++ decoder, {threads} threads over row ranges) + torch F.linear "
                            f"bf16 ({threads} threads) per call")
    torch.set_num_threads(1)
    per, reps, w = timed(lambda h: torch.nn.functional.linear(xcpu[h[4]], decode(h, 1)), host, 0.8 * budget_s, 1)
    legs["one_thread"] = leg("one_thread", per, w, reps, 1,
                             "decode (drinkme C++ decoder, one thread) + torch F.linear bf16 (one thread) per call")
    torch.set_num_threads(threads)
    weights = [(decode(h, threads), h[4]) for h in host]
    per, reps, w = timed(lambda wc: torch.nn.functional.linear(xcpu[wc[1]], wc[0]),
                         [(W, C, 0, W.shape[0], W.shape[1]) for W, C in weights], 0.4 * budget_s)
    legs["cached_w"] = leg("cached_w", per, w, reps, threads,
                           f"torch F.linear bf16 ({threads} threads) over the decoded weight, kept between calls")
    out = dict(legs["cpu_share"])
    out.update(kind=kind, legs=legs, nproc=nproc, affinity_cpus=allowed,
               threads_note=f"{threads} threads: the CPUs this process may run on ({allowed} of nproc {nproc}), "
                            f"at most {CPU_SHARE}, the host CPUs a one-GPU job is given")
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="qwen3-8b-step",
                    choices=["qwen3-8b-step", "qwen3-8b-layer", "32b-layer", "linear-4096"])
    ap.add_argument("--profile", default="sip", choices=["sip", "gulp", "balanced"])
    ap.add_argument("--m", type=int, default=1, choices=range(1, 9), help="activation rows (MTP verify: 4)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only the dominant kernel's graph (for counter passes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU; --gpus {args.gpus} is not supported (this build measures one "
              "GPU's share: the kernel is row-parallel, and a multi-GPU run would give each GPU its rows)",
              file=sys.stderr)
        return 2

    import torch

    from drinkme_amd import radix_ops, synth

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    items = workload_items(args.workload)
    if args.kernel_only:
        items = [it for it in items if it[2] in ("gate", "up")][:16] or items[:8]
    log(f"workload {args.workload}: {len(items)} GEMVs, profile {args.profile}")
    tensors = build_tensors(items, args.profile, args.m)
    xs = {}
    for c in sorted({t["C"] for t in tensors}):
        xb = synth.activation(args.workload, f"x{c}", args.m, c)
        xs[c] = torch.from_numpy(xb.view("int16")).view(torch.bfloat16).cuda()
    outs = [torch.empty((args.m, t["R"]), dtype=torch.bfloat16, device="cuda") for t in tensors]
    descs = [radix_ops.descriptor(t["rt"]) for t in tensors]

    import ctypes as ct

    from drinkme_amd import _native

    lib = _native.lib()
    err = _native.error_buffer()

    # launches: the GEMVs of a layer that share an activation go together
    share = {"q": "qkv", "k": "qkv", "v": "qkv", "gate": "gateup", "up": "gateup"}
    groups, last = [], None
    for i, t in enumerate(tensors):
        key = (t["layer"], share.get(t["name"]))
        if key[1] is not None and key == last:
            groups[-1].append(i)
        else:
            groups.append([i])
        last = key
    garrs = []
    for grp in groups:
        n = len(grp)
        garrs.append((n, (ct.POINTER(_native.RadixTensor) * n)(*[ct.pointer(descs[i]) for i in grp]),
                      (ct.c_void_p * n)(*[outs[i].data_ptr() for i in grp]), tensors[grp[0]]["C"]))

    def stream():
        return ct.c_void_p(torch.cuda.current_stream().cuda_stream)

    def launch_group(gi):
        n, tarr, oarr, C = garrs[gi]
        st = lib.dmx_radix_gemv_group(tarr, n, xs[C].data_ptr(), _native.DMX_BF16, args.m, None, 0, oarr,
                                      _native.DMX_BF16, stream(), err, len(err))
        if st:
            raise RuntimeError(err.value.decode())

    def launch(i):
        t = tensors[i]
        st = lib.dmx_radix_gemv(ct.byref(descs[i]), xs[t["C"]].data_ptr(), _native.DMX_BF16, args.m, None, 0,
                                outs[i].data_ptr(), _native.DMX_BF16, stream(), err, len(err))
        if st:
            raise RuntimeError(err.value.decode())

    def sweep():
        for gi in range(len(groups)):
            launch_group(gi)

    def sweep_ungrouped():
        for i in range(len(tensors)):
            launch(i)

    # the dominant launch: a layer's grouped gate/up (48% of the step's
    # weights; down is 24%, lm_head 8%), else the largest launch; timed over
    # every launch of the same tensors' shapes in the sweep
    gbytes = [sum(tensors[i]["bytes"] for i in grp) for grp in groups]
    sig = [tuple((tensors[i]["name"], tensors[i]["R"], tensors[i]["C"]) for i in grp) for grp in groups]
    pick = next((gi for gi, grp in enumerate(groups) if sorted(tensors[i]["name"] for i in grp) == ["gate", "up"]),
                gbytes.index(max(gbytes)))
    dom = [gi for gi in range(len(groups)) if sig[gi] == sig[pick]]
    dom_shape = " + ".join(f"{tensors[i]['R']}x{tensors[i]['C']}" for i in groups[dom[0]])

    def dominant():
        for gi in dom:
            launch_group(gi)

    total_bytes = sum(t["bytes"] for t in tensors)
    total_bf16 = sum(t["bf16_bytes"] for t in tensors)
    dom_info = {}
    dom_ms = time_graph(dominant, max(args.steps, 10), args.warmup, settle_s=0.3, info=dom_info)
    dom_bytes = sum(gbytes[gi] for gi in dom) / len(dom)
    dom_us = dom_ms * 1e3 / len(dom)
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9
    log(f"dominant launch {dom_shape}: {dom_us:.2f} us/launch, {achieved:.0f} GB/s ({achieved / PEAK_GBPS:.1%} of peak), "
        f"{round(dom_bytes)} algorithmic bytes per launch")
    if args.kernel_only:
        # a plain copy of known size beside it: the scale for counter-derived
        # bytes; then reductions over the same 256 MiB, a second scale for
        # the read counter from a kernel that only reads
        src = torch.empty(64 * 2**20, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration copy: 3 x 256 MiB device-to-device")
        for _ in range(3):
            src.sum()
        torch.cuda.synchronize()
        log("calibration read: 3 sums over 256 MiB")
        return 0
    ms = time_graph(sweep, args.steps, args.warmup)
    value = total_bytes / (ms * 1e-3) / 1e9
    log(f"sweep ({len(groups)} launches): {ms * 1e3:.1f} us, {value:.0f} GB/s compressed ({value / PEAK_GBPS:.1%}), "
        f"{total_bf16 / (ms * 1e-3) / 1e9:.0f} GB/s bf16-equivalent")
    # the same launches as plain reads of their bytes (dmx_read_probe, one
    # launch per launch of the sweep, each over a buffer of its own): the
    # ceiling for this sweep on this box, timed the same way
    wgs = 2 * torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.zeros(wgs, dtype=torch.int32, device="cuda")
    rbufs = [torch.empty((b + 15) // 16 * 4, dtype=torch.int32, device="cuda") for b in gbytes]

    def read_launch(buf):
        st = lib.dmx_read_probe(buf.data_ptr(), buf.numel() * 4, sink.data_ptr(), wgs, stream(), err, len(err))
        if st:
            raise RuntimeError(err.value.decode())

    def read_sweep():
        for buf in rbufs:
            read_launch(buf)

    big = max(rbufs, key=lambda b: b.numel())

    def read_big():
        for _ in range(4):
            read_launch(big)

    ms_r = time_graph(read_sweep, args.steps, args.warmup)
    read_bytes = sum(b.numel() * 4 for b in rbufs)
    big_gbps = 4 * big.numel() * 4 / (time_graph(read_big, args.steps, args.warmup) * 1e-3) / 1e9
    read_wall = {"us_per_sweep": round(ms_r * 1e3, 2), "value": round(read_bytes / (ms_r * 1e-3) / 1e9, 1),
                 "pct_of_hbm_peak": round(100 * read_bytes / (ms_r * 1e-3) / 1e9 / PEAK_GBPS, 2),
                 "sweep_fraction_of_read_wall": round(ms_r / ms, 4),
                 "largest_launch": {"bytes": big.numel() * 4, "value": round(big_gbps, 1)},
                 "kernel": f"dmx_read_probe: non-temporal 16-byte reads, {wgs} workgroups of 1024 threads, one launch "
                           "per launch of the sweep over its algorithmic bytes"}
    # per launch kind (the launches of one shape: a layer's q/k/v, o,
    # gate/up, down; lm_head), each kind's launches as a graph of their own:
    # the kernel against the plain read of the same buffers' bytes
    kinds = {}
    for gi, sg in enumerate(sig):
        kinds.setdefault(sg, []).append(gi)
    per_kind = {}
    for sg, gis in kinds.items():
        name = "+".join(n for n, _, _ in sg)

        def kernel_kind(gis=gis):
            for gi in gis:
                launch_group(gi)

        def read_kind(gis=gis):
            for gi in gis:
                read_launch(rbufs[gi])

        k_us = time_graph(kernel_kind, args.steps, args.warmup) * 1e3 / len(gis)
        r_us = time_graph(read_kind, args.steps, args.warmup) * 1e3 / len(gis)
        per_kind[name] = {"launches": len(gis), "bytes": round(sum(gbytes[gi] for gi in gis) / len(gis)),
                          "kernel_us": round(k_us, 2), "read_us": round(r_us, 2), "kernel_over_read": round(k_us / r_us, 3)}
    read_wall["per_launch_kind"] = per_kind
    del rbufs, big
    log(f"plain read of the same launches: {ms_r * 1e3:.1f} us, {read_wall['value']:.0f} GB/s "
        f"({read_wall['pct_of_hbm_peak']:.1f}% of peak); the sweep runs at {read_wall['sweep_fraction_of_read_wall']:.1%} "
        f"of it; the largest launch's bytes alone read at {big_gbps:.0f} GB/s")
    for name, pk in per_kind.items():
        log(f"  {name}: {pk['bytes'] / 1e6:.1f} MB, kernel {pk['kernel_us']:.2f} us, plain read {pk['read_us']:.2f} us "
            f"({pk['kernel_over_read']:.2f}x), {pk['launches']} launch(es) in its graph")
    # gulp's 3- and 4-row verify: AUTO runs it on v_dot2 (measured faster);
    # the matrix policy runs it in quad units on the matrix cores, as 8 rows
    # run: the same sweep timed on that path too
    matrix = None
    if args.profile == "gulp" and args.m in (3, 4):
        prev = radix_ops.set_policy("matrix")
        try:
            ms_mx = time_graph(sweep, args.steps, args.warmup)
        finally:
            radix_ops.set_policy(prev)
        matrix = {"us_per_sweep": round(ms_mx * 1e3, 2), "value": round(total_bytes / (ms_mx * 1e-3) / 1e9, 1),
                  "path": "radix_ops.set_policy('matrix'): the verify rows in quad units on the matrix cores "
                          "(v_mfma_f32_4x4x4_16b_bf16); the line's value is the default path, v_dot2"}
        log(f"sweep on the matrix cores (policy 'matrix'): {ms_mx * 1e3:.1f} us, {matrix['value']:.0f} GB/s compressed")
    ms_u = time_graph(sweep_ungrouped, args.steps, args.warmup)
    log(f"sweep ungrouped ({len(tensors)} launches): {ms_u * 1e3:.1f} us, "
        f"{total_bytes / (ms_u * 1e-3) / 1e9:.0f} GB/s compressed")
    # drinkme's own launch pattern: one call per Linear through the radix_ops
    # surface (gemv_fused at M = 1, the fused rows call above), eagerly on the
    # current stream, each call allocating its output (swap.py:443-456)
    def sweep_eager():
        for t in tensors:
            x = xs[t["C"]]
            if args.m == 1:
                radix_ops.gemv_fused(t["rt"], x[0], None, torch.bfloat16)
            else:
                radix_ops.gemv_rows(t["rt"], x, None, torch.bfloat16)

    ms_e, host_e = time_eager(sweep_eager, args.steps, args.warmup)
    log(f"sweep eager, one radix_ops call per Linear ({len(tensors)} launches): {ms_e * 1e3:.1f} us "
        f"({host_e * 1e3:.0f} us of host issue), {total_bytes / (ms_e * 1e-3) / 1e9:.0f} GB/s compressed")
    # the module surface as a decoder layer calls it: one RadixCompressedLinear
    # per Linear, called one by one on the layer's activation [1, M, C], with
    # the q/k/v and gate/up modules joined by SharedInputGroup (one grouped
    # launch each, the other members served from it), eagerly
    from drinkme_amd import swap

    mods = [swap.RadixCompressedLinear(t["rt"]) for t in tensors]
    for grp in groups:
        if len(grp) > 1:
            swap.SharedInputGroup([mods[i] for i in grp])
    xin = {c: x.reshape(1, args.m, c) for c, x in xs.items()}

    def sweep_modules():
        for mod, t in zip(mods, tensors):
            mod(xin[t["C"]])

    ms_md, host_md = time_eager(sweep_modules, args.steps, args.warmup)
    log(f"sweep eager, one module call per Linear, q/k/v and gate/up grouped ({len(groups)} launches): "
        f"{ms_md * 1e3:.1f} us ({host_md * 1e3:.0f} us of host issue), "
        f"{total_bytes / (ms_md * 1e-3) / 1e9:.0f} GB/s compressed")
    traffic = None
    tf = os.path.join(ROOT, "profiles", "traffic.json")
    key = f"k_gemv_{args.profile} {dom_shape} {args.profile} M={args.m}"
    if os.path.exists(tf):
        traffic = json.load(open(tf)).get(key, {}).get("hbm_bytes_per_launch")
    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        cpu = cpu_baseline(tensors, xs)
        for name, lg in cpu["legs"].items():
            log(f"cpu baseline {name}: {lg['value']:.3f} GB/s ({lg['ms_per_step']:.0f} ms per sweep, "
                f"{lg['cores']} thread(s))")
    out = {
        "metric": "compressed-HBM GB/s of the Qwen3-8B decode-step GEMV sweep (sip, M=1)"
        if (args.workload, args.profile, args.m) == ("qwen3-8b-step", "sip", 1)
        else f"compressed-HBM GB/s ({args.workload}, {args.profile}, M={args.m})",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": args.workload, "profile": args.profile, "m": args.m, "gemvs": len(tensors),
            "weights": sum(t["R"] * t["C"] for t in tensors), "compressed_bytes": total_bytes,
            "bpw": round(8 * total_bytes / sum(t["R"] * t["C"] for t in tensors), 4),
            "us_per_sweep": round(ms * 1e3, 2), "pct_of_hbm_peak": round(100 * value / PEAK_GBPS, 2),
            "effective_bf16_gbps": round(total_bf16 / (ms * 1e-3) / 1e9, 1),
            "launches": len(groups), "grouping": "q/k/v and gate/up of a layer share x: one launch each",
            "ungrouped": {"launches": len(tensors), "us_per_sweep": round(ms_u * 1e3, 2),
                          "value": round(total_bytes / (ms_u * 1e-3) / 1e9, 1)},
            "eager_ungrouped": {"launches": len(tensors), "us_per_sweep": round(ms_e * 1e3, 2),
                                "value": round(total_bytes / (ms_e * 1e-3) / 1e9, 1),
                                "host_issue_us_per_sweep": round(host_e * 1e3, 1),
                                "calls": "radix_ops.gemv_fused per Linear (gemv_rows at M > 1), eager, no graph"},
            "eager_modules": {"launches": len(groups), "us_per_sweep": round(ms_md * 1e3, 2),
                              "value": round(total_bytes / (ms_md * 1e-3) / 1e9, 1),
                              "host_issue_us_per_sweep": round(host_md * 1e3, 1),
                              "calls": "one RadixCompressedLinear call per Linear on x [1, M, C], q/k/v and gate/up "
                                       "joined by swap.SharedInputGroup, eager, no graph"},
            "read_wall": read_wall,
            "timing": "HIP graph of the sweep, replayed; events around the timed replays",
            **({"matrix_cores": matrix} if matrix else {}),
            "weights_rng": f"dmx_synth_bf16 seed {synth.SEED}, one stream per (workload, layer, tensor)",
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / PEAK_GBPS, 4), "traffic": traffic,
            "kernel": {"sip": "k_gemv_sip", "gulp": "k_gemv_gulp"}.get(args.profile, "k_gemv_generic"),
            "shape": dom_shape,
            "bytes_per_launch": round(dom_bytes), "us_per_launch": round(dom_us, 3),
            "launches_timed": len(dom), "settle_replays": dom_info["settle_replays"],
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
