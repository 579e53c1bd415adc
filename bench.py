#!/usr/bin/env python3
"""Benchmark of the tiered decode-attention path on one MI355X; prints one JSON line.

Default workload (`--workload decode128k`): the Llama-3.1-8B-shaped tiered decode step at
131,072 tokens and a 6.25% budget. Per decode step, 32 selecting layers: 32 query / 8 KV heads,
head_dim 128, bf16 KV, 16-token blocks, 8,192 blocks per KV head of which 8,190 are candidates;
K = 512 selected per KV head. Every layer's KV lives in mapped pinned host memory (512 MiB per
layer, 16 GiB in all); the block metadata, the sink and the current block live in HBM. Per
layer, one step runs the Quest bound + top-K kernels over the metadata and the block-sparse
decode kernels, which read the 4,096 selected (block, head) pairs in place over PCIe. Nothing
returns to the host between layers. The 32-layer step is captured once in a HIP graph and
replayed. `value` = decode-step microseconds per layer (lower is better); beside it the same step
with the KV resident in HBM, per-kernel durations against the byte roofline, the link probe, and
the reference's CPU decode path (`oracle/cpu_path.py`) timed on this host on a bounded sample.

Other workloads (same JSON contract, for the parity-test configurations):
  decode32k  -- Llama-3.2-1B-shaped decode, 32,768 tokens, d 64, float16, K 512, all in HBM
                (16 seeded layer instances, rotated so the 256 MB last-level cache cannot hold them)
  int8_64k   -- 1B-shaped, 16 layers, 65,536 tokens, d 64, float16, K 1,024, sealed blocks as int8
                records (`--tier-where hbm|host`), dequantised in the decode load
  exact128k  -- 8B-shaped exact split, 32 layers, 131,072 tokens: K of 512 / 2,048 / 4,096 from the
                exact HBM store, every other sealed block from the int8 host tier, merged by LSE
  prefill32k -- 1B-shaped layer-major prefill of a 32,768-token prompt, 16 layers, float16, every
                layer's KV turned into the int8 host tier by the fused pack + metadata kernel
  hybrid128k -- the 8B-shaped step over a sequence of decode steps whose queries drift (`--drift`):
                hybrid residency (HBM slots for the k most recently selected blocks per head, misses
                read in place and admitted) against the zero-copy read of the same sequence; the host
                tier holds bf16 pairs or, with `--quant int8`, int8 records

    python bench.py [--workload W] [--steps K] [--warmup W] [--layers L] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

DENSE_LAYERS = 2  # the reference's default dense layers, for the int8_64k variant that keeps them
METRIC = "decode-step µs/layer & achieved HBM GB/s (% roofline) at 128K ctx, 6.25% budget"
HBM_PEAK_GBPS = 8000.0
PCIE_PEAK_GBPS = 64.0  # PCIe Gen5 x16, one direction
N_Q, H, BS = 32, 8, 16
TRAFFIC_FILE = ROOT / "profiles" / "pmc_traffic.json"  # rocprofv3 FETCH_SIZE / WRITE_SIZE per kernel, every workload

WORKLOADS = {
    "decode128k": dict(layers=32, tokens=131072, d=128, dtype="bfloat16", k=(512,), kind="host"),
    "decode32k": dict(layers=16, tokens=32768, d=64, dtype="float16", k=(512,), kind="hbm"),
    "int8_64k": dict(layers=16, tokens=65536, d=64, dtype="float16", k=(1024,), kind="int8"),
    "exact128k": dict(layers=32, tokens=131072, d=128, dtype="bfloat16", k=(512, 2048, 4096), kind="exact"),
    "prefill32k": dict(layers=16, tokens=32768, d=64, dtype="float16", k=(512,), kind="prefill"),
    "hybrid128k": dict(layers=32, tokens=131072, d=128, dtype="bfloat16", k=(512,), kind="hybrid"),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--workload", choices=sorted(WORKLOADS), default="decode128k")
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--layers", type=int, default=None)
    p.add_argument("--tokens", type=int, default=None)
    p.add_argument("--k", type=int, default=None, help="selected blocks per KV head (default: the workload's)")
    p.add_argument("--block-size", type=int, default=16, choices=[16, 32, 64, 128, 256],
                   help="tokens per block; without --k the workload's K is scaled to keep its token budget")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--only", choices=["zerocopy", "hbm"], default=None, help="decode128k: one leg only")
    p.add_argument("--tier-where", choices=["hbm", "host"], default="hbm", help="int8_64k: where the int8 records live")
    p.add_argument("--eager", action="store_true", help="launch from Python instead of replaying a graph")
    p.add_argument("--unfused", action="store_true", help="the step as two calls (lkv_bound_topk, lkv_sparse_decode) instead of one (lkv_select_decode)")
    p.add_argument("--coherent", action="store_true", help="fine-grained (device-uncached) host pools")
    p.add_argument("--drift", type=float, default=0.25, help="hybrid128k: per-step query drift (relative to the query's RMS)")
    p.add_argument("--seq", type=int, default=16, help="hybrid128k: decode steps in the sequence")
    p.add_argument("--quant", choices=["none", "int8"], default="none", help="hybrid128k: host tier as model-dtype pairs or int8 records")
    args = p.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path has no multi-GPU mode (asked for --gpus {args.gpus}).", file=sys.stderr)
        return 2
    global BS
    BS = args.block_size
    spec = dict(WORKLOADS[args.workload])
    spec["layers"] = args.layers or spec["layers"]
    spec["tokens"] = args.tokens or spec["tokens"]
    if args.k:
        spec["k"] = (args.k,)
    elif BS != 16:
        spec["k"] = tuple(max(1, k * 16 // BS) for k in spec["k"])
    runners = {"prefill": run_prefill, "hybrid": run_hybrid}
    out = runners.get(spec["kind"], run_decode)(args, spec)
    print(json.dumps(out), flush=True)
    return 0


# -- shared timing --------------------------------------------------------------------------------


def _events(n: int):  # noqa: ANN202
    import torch

    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def time_step(step, steps: int, warmup: int, eager: bool) -> tuple[float, float, dict]:  # noqa: ANN001
    """(ms per step, wall s, per-step distribution): `step` captured once in a HIP graph and
    replayed, or launched eagerly. The first two figures time `steps` back-to-back steps between
    two events; the distribution then times at least 20 (up to 100, about 10 s) further steps
    each between events of its own, for the median and interquartile range."""
    import torch

    step()
    torch.cuda.synchronize()
    graph = None
    if not eager:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        torch.cuda.synchronize()
    run = graph.replay if graph is not None else step
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    e0, e1 = _events(2)
    wall0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        run()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = e0.elapsed_time(e1) / steps
    n = max(20, min(100, int(10_000 / max(ms, 1e-3))))
    ev = _events(n + 1)
    ev[0].record()
    for i in range(n):
        run()
        ev[i + 1].record()
    torch.cuda.synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(n)]
    q1, q2, q3 = statistics.quantiles(per, n=4)
    del graph
    return ms, wall, {"median_ms": q2, "iqr_ms": [q1, q3], "steps": n}


def kernel_us(calls: list, reps: int) -> list[float]:
    """Mean duration of each callable, launched eagerly, bracketed by events on the launch stream."""
    import torch

    marks = []
    for _ in range(reps):
        ev = _events(len(calls) + 1)
        ev[0].record()
        for i, c in enumerate(calls):
            c()
            ev[i + 1].record()
        marks.append(ev)
    torch.cuda.synchronize()
    return [statistics.mean(ev[i].elapsed_time(ev[i + 1]) for ev in marks) * 1e3 for i in range(len(calls))]


def graph_launch_us(calls: list, reps: int = 20) -> float:
    """Microseconds per launch of `calls` (independent launches, one per layer) captured back to back
    in one HIP graph and replayed `reps` times between two events: the launches' own durations plus
    the gap a graph leaves between dependent launches on one stream (about 1 us on MI355X), without
    the host's launch latency that an eager, event-bracketed call carries."""
    import torch

    for c in calls:
        c()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for c in calls:
            c()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = _events(2)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    del graph
    return e0.elapsed_time(e1) * 1e3 / (reps * len(calls))


def probe_gbps(addr: int, nbytes: int, blocks: int, reps: int = 5) -> float:
    """The link (or HBM) asymptote: a streaming read of `nbytes` at a device-visible address."""
    import torch

    from lazykv_amd import kernels

    sink = torch.zeros(4096, dtype=torch.int32, device="cuda")
    kernels.stream_read(addr, nbytes, blocks, sink)
    torch.cuda.synchronize()
    e0, e1 = _events(2)
    e0.record()
    for _ in range(reps):
        kernels.stream_read(addr, nbytes, blocks, sink)
    e1.record()
    torch.cuda.synchronize()
    return nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9


def dma_h2d_gbps(host, reps: int = 3) -> float:  # noqa: ANN001
    """The copy engines' host-to-device rate over the same pinned pool (a plain hipMemcpyAsync):
    the link's practical ceiling, to set the kernels' reads beside."""
    import torch

    src = host.reshape(-1).view(torch.uint8)[: 512 << 20]
    dst = torch.empty_like(src, device="cuda")
    dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    e0, e1 = _events(2)
    e0.record()
    for _ in range(reps):
        dst.copy_(src, non_blocking=True)
    e1.record()
    torch.cuda.synchronize()
    return src.numel() * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9


def dma_d2h_gbps(host, reps: int = 3) -> float:  # noqa: ANN001
    """The copy engines' device-to-host rate into the same pinned pool (a plain hipMemcpyAsync):
    the link's practical write ceiling, to set the kernels' writes to host memory beside."""
    import torch

    dst = host.reshape(-1).view(torch.uint8)[: 512 << 20]
    src = torch.zeros_like(dst, device="cuda")
    dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    e0, e1 = _events(2)
    e0.record()
    for _ in range(reps):
        dst.copy_(src, non_blocking=True)
    e1.record()
    torch.cuda.synchronize()
    return dst.numel() * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9


def _pmc_file() -> dict:
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def step_kernels(fused: bool, in_decode: bool, n_cand: int) -> str:
    """One layer's launches, as rocprof names them, by the library's dispatch rules: the matrix-core
    bound for a model-dtype query with aligned rows; the top K inside the decode launch when the
    fused call selects there, else select_block_kernel up to 8,192 candidates, select_kernel up to
    12,288 and select_stream_kernel beyond."""
    call = "one lkv_select_decode call: " if fused else "lkv_bound_topk + lkv_sparse_decode: "
    if fused and in_decode:
        return call + "bound_kernel_mf, sparse_decode_kernel choosing the top K itself, decode_merge_wave_kernel"
    sel = "select_block_kernel" if n_cand <= 8192 else ("select_kernel" if n_cand <= 12288 else "select_stream_kernel")
    return call + f"bound_kernel_mf, {sel}, sparse_decode_kernel, decode_merge_wave_kernel"


def pmc_traffic(workload: str) -> dict:
    """Calibrated HBM/fabric bytes per launch, per "<leg>/<kernel>", for `workload`, from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (a counter run cannot time itself, so
    separate runs of the same step supply them)."""
    prefix = workload + "/"
    return {key[len(prefix):]: v["traffic_bytes"] for key, v in _pmc_file().get("kernels", {}).items() if key.startswith(prefix)}


def pmc_run(workload: str, leg: str) -> str | None:
    """The profiler command whose counters `pmc_traffic` reports for a workload's leg."""
    return _pmc_file().get("runs", {}).get(f"{workload}/{leg}")


def cpu_cores() -> tuple[int, int]:
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return max(1, min(16, avail)), avail


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            return next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        return ""


def time_cpu(fn, states: list, budget_s: float) -> dict:  # noqa: ANN001
    """Median seconds of `fn(*state)` over rotating states, at 8 threads and at the core count."""
    import torch

    cores, avail = cpu_cores()
    settings = sorted({min(8, cores), cores})
    prev = torch.get_num_threads()
    results = {}
    for n in settings:
        torch.set_num_threads(n)
        fn(*states[0])  # warmup
        times, i, t_start = [], 0, time.perf_counter()
        while (time.perf_counter() - t_start) < budget_s / len(settings) or len(times) < 3:
            t0 = time.perf_counter()
            fn(*states[i % len(states)])
            times.append(time.perf_counter() - t0)
            i += 1
        results[n] = times
        log(f"cpu baseline, {n} threads: median {statistics.median(times) * 1e3:.2f} ms over {len(times)} runs")
    torch.set_num_threads(prev)
    t = results[cores]
    med = statistics.median(t)
    q1, _, q3 = statistics.quantiles(t, n=4) if len(t) >= 4 else (med, med, med)
    return {"median_s": med, "iqr_s": [q1, q3], "cores": cores, "avail": avail, "runs": sum(len(v) for v in results.values()),
            "runs_at_cores": len(t), "per_thread_setting_us": {str(n): round(statistics.median(v) * 1e6, 1) for n, v in results.items()}}


# -- decode workloads -----------------------------------------------------------------------------


def run_decode(args: argparse.Namespace, spec: dict) -> dict:
    import torch

    from lazykv_amd import kernels
    from lazykv_amd.pinned import device_address, pinned_empty
    from lazykv_amd.quant import packed_pair_bytes
    from lazykv_amd.workload import draw_layer, to_pool

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    dtype = getattr(torch, spec["dtype"])
    d, T, L, kind, ks = spec["d"], spec["tokens"], spec["layers"], spec["kind"], spec["k"]
    N = T // BS
    n_sealed, fill = N - 1, BS  # lazy sealing: the last block is the current one, full
    n_cand = n_sealed - 1
    scale = d**-0.5
    es = torch.tensor([], dtype=dtype).element_size()
    P = packed_pair_bytes(BS, d)
    want_host = kind == "host" and args.only in (None, "zerocopy")
    want_hbm_leg = kind == "hbm" or (kind == "host" and args.only in (None, "hbm"))

    # ---- state ---------------------------------------------------------------------------------
    t0 = time.time()
    layers = []
    for li in range(L):
        w = draw_layer(li, N_Q, H, d, T, BS, dtype, device=dev)
        pool = to_pool(w.keys, w.values, BS)  # [N, h, 2, bs, d] on the GPU
        kmin = torch.zeros((1, H, N, d), dtype=dtype, device=dev)
        kmax = torch.zeros_like(kmin)
        src = kernels.dense_source(w.keys, w.values, BS)
        st = {"q": w.query.contiguous(), "kmin": kmin, "kmax": kmax, "slots": pool[[0, N - 1]].contiguous(), "needle": w.needle}
        if kind == "int8":
            recs = torch.zeros((N, H, P), dtype=torch.uint8, device=dev) if args.tier_where == "hbm" else pinned_empty((N, H, P), torch.uint8)
            # The records and the metadata of their dequantised keys, in one pass.
            kernels.store_blocks(src, dst=kernels.record_source(recs, dtype), n_kv=H, head_dim=d, block_size=BS, first_block=0, n_blocks=n_sealed, kmin=kmin, kmax=kmax)
            st["records"] = recs
        else:
            kernels.store_blocks(src, n_kv=H, head_dim=d, block_size=BS, first_block=0, n_blocks=n_sealed, kmin=kmin, kmax=kmax)
        if kind == "exact":
            recs = pinned_empty((N, H, P), torch.uint8)
            kernels.store_blocks(src, dst=kernels.record_source(recs, dtype), n_kv=H, head_dim=d, block_size=BS, first_block=0, n_blocks=n_sealed)
            st["records"] = recs
        if want_host:
            host = pinned_empty(tuple(pool.shape), dtype, coherent=args.coherent)
            host.copy_(pool)
            st["host"] = host
        if want_hbm_leg or kind == "exact":
            st["pool"] = pool
        if kind == "int8" and li < DENSE_LAYERS:  # the 2-dense variant keeps these layers' full KV in HBM
            st["dense"] = (w.keys, w.values)
        del w, pool, src
        layers.append(st)
        if li % 8 == 7:
            log(f"built {li + 1}/{L} layers ({time.time() - t0:.1f}s)")
    torch.cuda.synchronize()
    log(f"state ready in {time.time() - t0:.1f}s: {L} layers x {N} blocks, kind {kind}")

    # ---- legs: (name, k, selected source per layer, remainder source per layer or None) -----------
    legs = []
    if kind == "host":
        if want_host:
            legs.append(("zerocopy", ks[0], [kernels.pool_source(st["host"]) for st in layers], None))
        if want_hbm_leg:
            legs.append(("hbm", ks[0], [kernels.pool_source(st["pool"]) for st in layers], None))
    elif kind == "hbm":
        legs.append(("hbm", ks[0], [kernels.pool_source(st["pool"]) for st in layers], None))
    elif kind == "int8":
        legs.append((f"int8_{args.tier_where}", ks[0], [kernels.record_source(st["records"], dtype) for st in layers], None))
        # The reference's default keeps the first two layers dense (lazykv/selection.py:35): those
        # layers attend all their tokens from HBM, the other 14 select from the int8 tier.
        legs.append((f"int8_{args.tier_where}_{DENSE_LAYERS}dense", ks[0], [kernels.record_source(st["records"], dtype) for st in layers], None))
    else:
        for k in ks:
            legs.append((f"exact_k{k}", k, [kernels.pool_source(st["pool"]) for st in layers], [kernels.record_source(st["records"], dtype) for st in layers]))

    outs = [torch.empty((N_Q, d), dtype=dtype, device=dev) for _ in range(L)]
    lses = [torch.empty((N_Q,), dtype=torch.float32, device=dev) for _ in range(L)]
    ws_sel, ws_dec = kernels.Workspace(dev), kernels.Workspace(dev)
    res = {}
    for name, k, sels, rems in legs:
        n_dense = DENSE_LAYERS if name.endswith("dense") else 0
        idx = torch.empty((H, k), dtype=torch.int32, device=dev)
        ranks, decodes, checks = [], [], []
        fused = not args.unfused and rems is None
        for li, st in enumerate(layers):
            if li < n_dense:  # dense decode: every block of the layer's KV, from HBM
                dsrc = kernels.dense_source(st["dense"][0], st["dense"][1], BS)
                ranks.append(None)
                checks.append(None)
                decodes.append(kernels.PreparedDecode(st["q"], n_kv=H, block_size=BS, scale=scale, sel=None, idx=None, sink=None, sink_block=-1, cur=None, cur_block=-1,
                                                      fill=0, out=outs[li], lse=lses[li], rem=dsrc, rem_range=(0, N), attend_selected=False, ws=ws_dec))
                continue
            ss = kernels.pool_source(st["slots"])
            if fused:
                # One call per layer (lkv_select_decode). For the per-kernel split, "rank" is what
                # runs before the decode launch: the bound kernel, and the top-K launch when the
                # selection is not made inside the decode launch.
                common = dict(cand_offset=1, n_cand=n_cand, block_size=BS, scale=scale, sel=sels[li], sink=ss, sink_block=0, cur=ss, cur_block=1,
                              fill=fill, out=outs[li], lse=lses[li], ws=ws_dec)
                decodes.append(kernels.PreparedSelectDecode(st["q"], st["kmin"], st["kmax"], k, **common))
                checks.append(kernels.PreparedSelectDecode(st["q"], st["kmin"], st["kmax"], k, out_idx=idx, **common))
                if not kernels._lib.selects_in_decode(n_cand, bool(sels[li].flags), N_Q // H):
                    ranks.append(kernels.PreparedBoundTopk(st["q"], st["kmin"], st["kmax"], k, cand_offset=1, n_cand=n_cand, out_idx=idx, ws=ws_sel))
                else:
                    bnd = torch.empty((H, n_cand), dtype=torch.float32, device=dev)
                    ranks.append(kernels.PreparedBoundTopk(st["q"], st["kmin"], st["kmax"], 0, cand_offset=1, n_cand=n_cand, out_bound=bnd, ws=ws_sel))
                continue
            ranks.append(kernels.PreparedBoundTopk(st["q"], st["kmin"], st["kmax"], k, cand_offset=1, n_cand=n_cand, out_idx=idx, ws=ws_sel))
            checks.append(None)
            extra = dict(rem=rems[li], rem_range=(1, n_sealed)) if rems is not None else {}
            decodes.append(kernels.PreparedDecode(st["q"], n_kv=H, block_size=BS, scale=scale, sel=sels[li], idx=idx, sink=ss, sink_block=0, cur=ss, cur_block=1,
                                                  fill=fill, out=outs[li], lse=lses[li], ws=ws_dec, **extra))

        def step(ranks=ranks, decodes=decodes, fused=fused) -> None:  # noqa: ANN001
            for rk, dc in zip(ranks, decodes):
                if rk is not None and not fused:
                    rk()
                dc()

        # Every selecting layer's needle is selected for every KV head; outputs are finite.
        for li in range(L):
            if ranks[li] is not None:
                if checks[li] is not None:
                    checks[li]()
                else:
                    ranks[li]()
                got = idx.cpu()
                assert (got == layers[li]["needle"]).any(dim=1).all(), f"layer {li}: needle block {layers[li]['needle']} not selected"
            decodes[li]()
        torch.cuda.synchronize()
        assert all(torch.isfinite(o.float()).all() for o in outs), "non-finite output"
        ms_step, wall, dist = time_step(step, args.steps, args.warmup, args.eager)
        reps = max(2, min(5, args.steps))
        per = [kernel_us([ranks[li], decodes[li]], reps) for li in range(n_dense, L)]
        sel_us = statistics.mean(x[0] for x in per)
        dec_us = statistics.mean(x[1] for x in per)
        if fused:  # the one call holds the bound (and top-K) launches too: the decode launch is the rest
            dec_us = max(dec_us - sel_us, 1e-3)
        dense_us = statistics.mean(kernel_us([decodes[li]], reps)[0] for li in range(n_dense)) if n_dense else None
        # The bound launch alone, as the step runs it: every selecting layer's bound launch back to
        # back in one graph (bounds only, into a scratch row per layer).
        bnds = [torch.empty((H, n_cand), dtype=torch.float32, device=dev) for _ in range(n_dense, L)]
        bound_only = [kernels.PreparedBoundTopk(layers[li]["q"], layers[li]["kmin"], layers[li]["kmax"], 0, cand_offset=1, n_cand=n_cand, out_bound=bnds[li - n_dense], ws=ws_sel)
                      for li in range(n_dense, L)]
        bound_graph_us = graph_launch_us(bound_only)
        del bound_only, bnds
        extra = f", dense decode {dense_us:.1f} us on {n_dense} layers" if n_dense else ""
        log(f"{name}: {ms_step:.3f} ms/step = {ms_step * 1e3 / L:.1f} us/layer (bound+topk {sel_us:.1f} us, decode {dec_us:.1f} us{extra}), wall {wall:.2f}s")
        res[name] = {"k": k, "ms_step": ms_step, "us_layer": ms_step * 1e3 / L, "sel_us": sel_us, "dec_us": dec_us, "host_sel": bool(sels[0].flags), "rem": rems is not None,
                     "dist": dist, "n_dense": n_dense, "dense_us": dense_us, "fused": fused, "bound_graph_us": bound_graph_us}

    # ---- ranking precision ------------------------------------------------------------------------
    # The step ranks on the float32 bound. The reference's tier ranks on the bound rounded to the
    # model dtype (top_blocks with dtype=None), whose 2^-8 (bf16) or 2^-11 (f16) relative steps tie
    # blocks near the K-th place. The share of each head's K blocks both rankings select, over
    # the first layers of this workload:
    common = []
    for st in layers[: min(L, 8)]:
        a = kernels.bound_topk(st["q"], st["kmin"], st["kmax"], ks[0], cand_offset=1, n_cand=n_cand, rank_mode=kernels._lib.RANK_F32).cpu().numpy()
        b = kernels.bound_topk(st["q"], st["kmin"], st["kmax"], ks[0], cand_offset=1, n_cand=n_cand, rank_mode=kernels._lib.RANK_MODEL).cpu().numpy()
        common.extend(len(set(a[j].tolist()) & set(b[j].tolist())) / ks[0] for j in range(H))
    rank_agreement = {"mean": round(statistics.mean(common), 4), "min": round(min(common), 4), "heads": len(common)}
    log(f"selected-set agreement, float32 against model-dtype ranking: {rank_agreement}")

    # ---- probes --------------------------------------------------------------------------------
    probe = {}
    host_buf = None
    for st in layers:
        if "host" in st:
            host_buf = st["host"]
        elif "records" in st and not st["records"].is_cuda:
            host_buf = st["records"]
        if host_buf is not None:
            break
    if host_buf is not None:
        probe["pcie_read_gbps"] = probe_gbps(device_address(host_buf), host_buf.numel() * host_buf.element_size() // 16 * 16, 2048)
        probe["dma_h2d_gbps"] = dma_h2d_gbps(host_buf)
    big = torch.empty(4 << 30, dtype=torch.uint8, device=dev)
    probe["hbm_read_gbps"] = probe_gbps(big.data_ptr(), big.numel(), 4096)
    del big
    log(f"probes: {probe}")

    # ---- bytes per layer, roofline -------------------------------------------------------------
    B_meta = 2 * H * n_cand * d * es
    B_q = N_Q * d * es
    B_out = N_Q * d * es + 4 * N_Q
    B_sinkcur = 2 * H * 2 * BS * d * es

    def leg_bytes(rr: dict) -> tuple[int, int, int, int]:
        """(selected bytes, remainder bytes, HBM bytes per layer, PCIe bytes per layer); with dense
        layers, the step's bytes averaged over its layers."""
        k = rr["k"]
        b_sel = H * k * P if kind == "int8" else 2 * H * k * BS * d * es
        b_rem = H * (n_cand - k) * P if rr["rem"] else 0
        hbm = B_meta + 2 * B_q + B_out + B_sinkcur + (0 if rr["host_sel"] else b_sel)
        pcie = (b_sel if rr["host_sel"] else 0) + b_rem
        nd = rr["n_dense"]
        if nd:
            dense = 2 * H * N * BS * d * es + B_q + B_out  # all K and V of the layer
            hbm = ((L - nd) * hbm + nd * dense) // L
            pcie = (L - nd) * pcie // L
        return b_sel, b_rem, hbm, pcie

    legs_out = {}
    for name, rr in res.items():
        b_sel, b_rem, hb, pb = leg_bytes(rr)
        t_roof = max(hb / (HBM_PEAK_GBPS * 1e9), pb / (PCIE_PEAK_GBPS * 1e9)) * 1e6
        bw_probe = probe.get("pcie_read_gbps")
        t_probe = max(hb / (HBM_PEAK_GBPS * 1e9), pb / (bw_probe * 1e9)) * 1e6 if (bw_probe and pb) else None
        dec_pcie = (b_sel if rr["host_sel"] else 0) + b_rem
        dec_hbm = B_sinkcur + B_q + B_out + (0 if rr["host_sel"] else b_sel)
        legs_out[name] = {
            "k": rr["k"], "us_per_layer": round(rr["us_layer"], 3), "ms_per_step": round(rr["ms_step"], 4), "fused": rr["fused"],
            "step_stats": {"us_per_layer_median": round(rr["dist"]["median_ms"] * 1e3 / L, 2),
                           "us_per_layer_iqr": [round(x * 1e3 / L, 2) for x in rr["dist"]["iqr_ms"]], "steps": rr["dist"]["steps"]},
            "hbm_bytes_per_layer": hb, "pcie_bytes_per_layer": pb,
            "t_roof_us": round(t_roof, 3), "frac": round(t_roof / rr["us_layer"], 4),
            "t_roof_us_at_probe": round(t_probe, 2) if t_probe else None, "frac_at_probe": round(t_probe / rr["us_layer"], 4) if t_probe else None,
            "bound_topk_us": round(rr["sel_us"], 2), "bound_topk_gbps": round((B_meta + B_q) / (rr["sel_us"] * 1e-6) / 1e9, 1),
            "bound_graph_us": round(rr["bound_graph_us"], 2), "bound_graph_gbps": round((B_meta + B_q) / (rr["bound_graph_us"] * 1e-6) / 1e9, 1),
            "sparse_decode_us": round(rr["dec_us"], 2), "sparse_decode_pcie_bytes": dec_pcie, "sparse_decode_hbm_bytes": dec_hbm,
            "sparse_decode_pcie_gbps": round(dec_pcie / (rr["dec_us"] * 1e-6) / 1e9, 2) if dec_pcie else None,
            "sparse_decode_hbm_gbps": round(dec_hbm / (rr["dec_us"] * 1e-6) / 1e9, 1),
        }
        if rr["n_dense"]:
            dense_bytes = 2 * H * N * BS * d * es
            legs_out[name].update(dense_layers=rr["n_dense"], dense_decode_us=round(rr["dense_us"], 2),
                                  dense_decode_hbm_gbps=round(dense_bytes / (rr["dense_us"] * 1e-6) / 1e9, 1))

    main_leg = next(iter(res))
    m = legs_out[main_leg]
    names = {
        "host": f"Llama-3.1-8B-shaped tiered decode step: {L} selecting layers, {T} tokens, {BS}-token blocks, K={m['k']} of {n_cand} candidates per KV head ({100 * m['k'] * BS / T:g}% budget), bf16 KV in mapped pinned host memory",
        "hbm": f"Llama-3.2-1B-shaped decode layer: {T} tokens, d {d}, float16, {BS}-token blocks, K={m['k']} of {n_cand} candidates per KV head, all in HBM ({L} rotated layer instances)",
        "int8": f"Llama-3.2-1B-shaped decode step: {L} selecting layers, {T} tokens, d {d}, float16, K={m['k']} of {n_cand} per KV head, sealed blocks as int8 records in {'HBM' if args.tier_where == 'hbm' else 'mapped host memory'}, dequantised on load",
        "exact": f"Llama-3.1-8B-shaped exact tiered decode step: {L} layers, {T} tokens, bf16, K of {n_cand} from the exact HBM store, every other sealed block from the int8 host tier, merged by LSE",
    }
    out = {
        "metric": METRIC if kind == "host" else f"{kind} decode-step µs/layer & achieved GB/s (% byte roofline)",
        "value": m["us_per_layer"],
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": m["ms_per_step"],
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if dtype == torch.bfloat16 else "f16",
        "data": "synthetic",
        "config": {
            "workload": names[kind],
            "layers": L, "tokens": T, "q_heads": N_Q, "kv_heads": H, "head_dim": d, "block_size": BS, "k": m["k"],
            "rank_dtype": "float32",
            "rank_note": "the reference's tier ranks on the bound rounded to the model dtype (top_blocks dtype=None), whose resolution (2^-8 relative for bf16, "
                         "2^-11 for f16) ties blocks near the K-th place; this step ranks on the float32 bound. rank_model_set_agreement is the measured share "
                         "of each head's K blocks that both rankings select on this workload (first 8 layers); the model-dtype ranking is available "
                         "(rank_dtype=None)",
            "rank_model_set_agreement": rank_agreement,
            "dense_layers": 0, "launch": "eager" if args.eager else "hip_graph",
            "launches_per_layer": 3 if (m["fused"] and kernels._lib.selects_in_decode(n_cand, res[main_leg]["host_sel"], N_Q // H)) else 4,
            "step_kernels": step_kernels(m["fused"], kernels._lib.selects_in_decode(n_cand, res[main_leg]["host_sel"], N_Q // H), n_cand),
            "host_memory": "fine-grained" if args.coherent else "coarse-grained",
        },
        "host_syncs_per_layer": 0,
        "step_stats": dict(m["step_stats"], note="each step replayed between events of its own, after the timed region"),
    }
    # The dominant kernel is lkv_sparse_decode: sparse_decode_kernel and its merge launch (the one-wave
    # merge up to 64 partials per head; the exact split's 100-odd partials take decode_merge_kernel).
    merge = "decode_merge_kernel" if kind == "exact" else "decode_merge_wave_kernel"
    traffic = pmc_traffic(args.workload)
    traffic_note = {}
    if traffic.get(f"{main_leg}/sparse_decode_kernel"):
        traffic_note = {"traffic_note": "calibrated FETCH_SIZE + WRITE_SIZE bytes per launch, host (PCIe) and HBM fetches together; algorithmic total incl. HBM part "
                                        f"{m['sparse_decode_pcie_bytes'] + m['sparse_decode_hbm_bytes']}; source {TRAFFIC_FILE.relative_to(ROOT)}",
                        "traffic_run": pmc_run(args.workload, main_leg)}
    if m["sparse_decode_pcie_bytes"]:
        gbps = m["sparse_decode_pcie_gbps"]
        kname = (f"sparse_decode_kernel (top-K inside) + {merge}" if (m["fused"] and kernels._lib.selects_in_decode(n_cand, res[main_leg]["host_sel"], N_Q // H))
                 else f"sparse_decode_kernel + {merge}")
        out["roofline"] = {"bound": "pcie", "kernel": f"{kname}, host reads over PCIe", "achieved": gbps,
                           "peak": PCIE_PEAK_GBPS, "unit": "GB/s", "frac": round(gbps / PCIE_PEAK_GBPS, 4), "traffic": traffic.get(f"{main_leg}/sparse_decode_kernel"),
                           "algorithmic_bytes": m["sparse_decode_pcie_bytes"], "kernel_us": m["sparse_decode_us"], **traffic_note}
        if probe.get("dma_h2d_gbps"):
            out["roofline"]["link_ceiling_gbps"] = round(probe["dma_h2d_gbps"], 2)  # the copy engines over the same pool
            out["roofline"]["frac_of_link_ceiling"] = round(gbps / probe["dma_h2d_gbps"], 4)
    else:
        gbps = m["sparse_decode_hbm_gbps"]
        kname = (f"sparse_decode_kernel (top-K inside) + {merge}" if (m["fused"] and kernels._lib.selects_in_decode(n_cand, res[main_leg]["host_sel"], N_Q // H))
                 else f"sparse_decode_kernel + {merge}")
        out["roofline"] = {"bound": "hbm", "kernel": f"{kname}, HBM", "achieved": gbps,
                           "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": traffic.get(f"{main_leg}/sparse_decode_kernel"),
                           "algorithmic_bytes": m["sparse_decode_hbm_bytes"], "kernel_us": m["sparse_decode_us"], **traffic_note}
    out["byte_roofline"] = {"hbm_bytes_per_layer": m["hbm_bytes_per_layer"], "pcie_bytes_per_layer": m["pcie_bytes_per_layer"],
                            "t_roof_us_at_64gbps": m["t_roof_us"], "frac_at_64gbps": m["frac"],
                            "t_roof_us_at_probe": m["t_roof_us_at_probe"], "frac_at_probe": m["frac_at_probe"]}
    out["kernels"] = {"bound": {"us_per_launch": m["bound_graph_us"], "hbm_bytes": B_meta + B_q, "gbps": m["bound_graph_gbps"],
                                "frac_hbm_peak": round(m["bound_graph_gbps"] / HBM_PEAK_GBPS, 4),
                                "method": f"the {L} layers' bound launches back to back in one HIP graph, replayed; per launch, including the graph's "
                                          "dependent-launch gap (about 1 us); the profiler's kernel-only average is in profiles/"},
                      "bound_topk_launch_inclusive": {"us": m["bound_topk_us"], "hbm_bytes": B_meta + B_q,
                                                      "note": "eager bound (+ top-K when it has its own launch) bracketed by events, host launch latency and "
                                                              "gaps included: a launch-inclusive figure, not the kernels' HBM rate"},
                      "sparse_decode": {"us": m["sparse_decode_us"], "pcie_bytes": m["sparse_decode_pcie_bytes"], "hbm_bytes": m["sparse_decode_hbm_bytes"],
                                        "pcie_gbps": m["sparse_decode_pcie_gbps"], "hbm_gbps": m["sparse_decode_hbm_gbps"]}}
    if kind == "host" and "hbm" in legs_out:
        hb = legs_out["hbm"]
        out["hbm_resident"] = {"us_per_layer": hb["us_per_layer"], "ms_per_step": hb["ms_per_step"], "hbm_bytes_per_layer": hb["hbm_bytes_per_layer"],
                               "decode_traffic": traffic.get("hbm/sparse_decode_kernel"),
                               "t_roof_us": hb["t_roof_us"], "frac": hb["frac"], "bound_us_per_launch": hb["bound_graph_us"], "bound_gbps": hb["bound_graph_gbps"],
                               "bound_topk_launch_inclusive_us": hb["bound_topk_us"],
                               "sparse_decode_us": hb["sparse_decode_us"], "sparse_decode_gbps": hb["sparse_decode_hbm_gbps"]}
        if main_leg == "hbm":
            out["config"]["workload"] = out["config"]["workload"].replace("bf16 KV in mapped pinned host memory", "bf16 KV resident in HBM")
    if len(legs_out) > 1 and kind != "host":
        out["legs"] = legs_out
    out["probes"] = {kk: round(v, 2) for kk, v in probe.items()}

    # ---- CPU baseline: the reference's path for this workload on this host's cores ---------------
    if not args.no_cpu_baseline:
        # Layer 0 decoded once more by the main leg's kernels, with a float32 output for the parity
        # figure beside the timing, and with the model-dtype output the timed steps write (not the
        # last leg's layer 0: in the reference's 2-dense variant that layer is dense).
        name0, k0, sels0, rems0 = legs[0]
        st0 = layers[0]
        ss0 = kernels.pool_source(st0["slots"])

        def layer0(out_dtype: torch.dtype) -> tuple:
            if res[name0]["fused"]:
                return kernels.select_decode(st0["q"], st0["kmin"], st0["kmax"], k0, cand_offset=1, n_cand=n_cand, block_size=BS, scale=scale, sel=sels0[0],
                                             sink=ss0, sink_block=0, cur=ss0, cur_block=1, fill=fill, out_dtype=out_dtype)
            idx0 = kernels.bound_topk(st0["q"], st0["kmin"], st0["kmax"], k0, cand_offset=1, n_cand=n_cand)
            extra0 = dict(rem=rems0[0], rem_range=(1, n_sealed)) if rems0 is not None else {}
            return kernels.sparse_decode(st0["q"], n_kv=H, block_size=BS, scale=scale, sel=sels0[0], idx=idx0, sink=ss0, sink_block=0, cur=ss0, cur_block=1,
                                         fill=fill, out_dtype=out_dtype, **extra0)

        f32, md = layer0(torch.float32), layer0(st0["slots"].dtype)
        torch.cuda.synchronize()
        out["cpu_baseline"] = cpu_baseline_decode(kind, layers, ks[0], n_sealed, fill, scale, args.cpu_seconds, (name0, k0, f32, md))
    return out


def cpu_baseline_decode(kind: str, layers: list, k: int, n_sealed: int, fill: int, scale: float, budget_s: float, layer0: tuple) -> dict:
    from oracle import cpu_path

    n_layers = min(len(layers), 2 if kind == "exact" else 8)
    states, fn = [], None
    for st in layers[:n_layers]:
        sink, cur = st["slots"][0].cpu(), st["slots"][1].cpu()
        q, kmin, kmax = st["q"].cpu(), st["kmin"].cpu(), st["kmax"].cpu()
        if kind == "host":
            fn = cpu_path.decode_layer
            states.append((q, kmin, kmax, n_sealed, k, st["host"], sink, cur, fill, scale))
        elif kind == "hbm":
            fn = cpu_path.decode_layer
            states.append((q, kmin, kmax, n_sealed, k, st["pool"].cpu(), sink, cur, fill, scale))
        elif kind == "int8":
            fn = cpu_path.decode_layer_int8
            states.append((q, kmin, kmax, n_sealed, k, st["records"].cpu(), sink, cur, fill, scale))
        else:
            fn = cpu_path.exact_layer
            pool = st["pool"].cpu()
            hh, bs, d = pool.shape[1], pool.shape[3], pool.shape[-1]
            mk = pool[:n_sealed, :, 0].permute(1, 0, 2, 3).reshape(hh, n_sealed * bs, d).float().contiguous()
            mv = pool[:n_sealed, :, 1].permute(1, 0, 2, 3).reshape(hh, n_sealed * bs, d).float().contiguous()
            states.append((q, kmin, kmax, n_sealed, k, pool, mk, mv, cur, fill, scale))
    # Parity beside the timing: the CPU path's layer-0 output and LSE against the GPU's. The
    # float32-output decode is the figure held to the 2e-3 bar; the timed model-dtype output also
    # carries its own rounding (one step of the output dtype, 2^-8 of |out| for bfloat16).
    r0 = fn(*states[0])
    leg, k0, (o32, l32), (omd, _) = layer0
    parity, diff = {}, None
    if k0 == k:
        parity = {"gpu_vs_cpu_layer0_max_abs_out_f32": float((r0[0] - o32.cpu()).abs().max()),
                  "gpu_vs_cpu_layer0_max_abs_lse": float((r0[1] - l32.cpu()).abs().max()),
                  "parity_leg": leg, "parity_bar": 2e-3}
        diff = float((r0[0] - omd.float().cpu()).abs().max())
    t = time_cpu(fn, states, budget_s)
    samples = {"host": "single-layer decodes: fp32 quest bound, topk, index_select gather from the host pool, cat, masked fp32 attention + logsumexp",
               "hbm": "single-layer decodes: fp32 quest bound, topk, index_select gather, cat, masked fp32 attention + logsumexp",
               "int8": "single-layer decodes: fp32 quest bound, topk, gather of int8 records, quant.py unpack, cat, masked fp32 attention + logsumexp",
               "exact": f"single-layer exact decodes at K={k}: the gathered partial as in decode, the batched masked CPU partial over the float32 mirror of every sealed block, LSE merge"}
    return {
        "value": round(t["median_s"] * 1e6, 1), "unit": "us/layer", "cores": t["cores"], "kind": "port",
        "sample": f"{t['runs']} {samples[kind]} (layers 0-{n_layers - 1} of the same workload; median over {t['runs_at_cores']} at {t['cores']} threads), torch CPU ops in the reference's order",
        "iqr_us": [round(x * 1e6, 1) for x in t["iqr_s"]], "per_thread_setting_us": t["per_thread_setting_us"],
        "cpu_model": cpu_model(), "host_cpus_visible": t["avail"], **parity,
        "gpu_vs_cpu_layer0_max_abs_out_model_dtype": diff,
        "model_dtype_note": "the timed decode writes the model dtype; its deviation includes that output's rounding (bfloat16: up to 2^-8 of |out|)",
    }


# -- hybrid residency over a drifting decode sequence ---------------------------------------------------


def run_hybrid(args: argparse.Namespace, spec: dict) -> dict:
    import torch

    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty
    from lazykv_amd.quant import packed_pair_bytes
    from lazykv_amd.workload import draw_layer, to_pool

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    dtype = getattr(torch, spec["dtype"])
    d, T, L, k = spec["d"], spec["tokens"], spec["layers"], spec["k"][0]
    N = T // BS
    n_sealed, fill, n_cand = N - 1, BS, N - 2
    S = max(2, args.seq)
    int8 = args.quant == "int8"
    t0 = time.time()
    layers = []
    for li in range(L):
        w = draw_layer(li, N_Q, H, d, T, BS, dtype, device=dev)
        pool = to_pool(w.keys, w.values, BS)
        kmin = torch.zeros((1, H, N, d), dtype=dtype, device=dev)
        kmax = torch.zeros_like(kmin)
        dense = kernels.dense_source(w.keys, w.values, BS)
        if int8:  # records packed into the host pool; metadata over the dequantised keys
            host = pinned_empty((N, H, packed_pair_bytes(BS, d)), torch.uint8)
            hs = kernels.record_source(host, dtype)
            kernels.store_blocks(dense, dst=hs, n_kv=H, head_dim=d, block_size=BS, first_block=0, n_blocks=n_sealed, kmin=kmin, kmax=kmax)
        else:
            kernels.store_blocks(dense, n_kv=H, head_dim=d, block_size=BS, first_block=0, n_blocks=n_sealed, kmin=kmin, kmax=kmax)
            host = pinned_empty(tuple(pool.shape), dtype)
            host.copy_(pool)
            hs = kernels.pool_source(host)
        layers.append({"q": w.query.float(), "kmin": kmin, "kmax": kmax, "slots": pool[[0, N - 1]].contiguous(), "host": host, "hs": hs,
                       "res": kernels.Residency.allocate(k, H, N, BS, d, dtype, dev)})
        del w, pool
    # The query sequence: each step's query is the layer's base query plus a fresh drift.
    gen = torch.Generator(device=dev).manual_seed(7)
    base = torch.stack([st["q"] for st in layers])  # [L, n_q, d] float32
    rms = base.pow(2).mean(dim=-1, keepdim=True).sqrt()
    q_seq = (base[None] + args.drift * rms[None] * torch.randn((S, *base.shape), generator=gen, device=dev)).to(dtype)
    q_static = torch.empty(base.shape, dtype=dtype, device=dev)
    torch.cuda.synchronize()
    log(f"state ready in {time.time() - t0:.1f}s: {L} layers x {N} blocks, {S} steps, drift {args.drift}")

    ws_h, ws_z = kernels.Workspace(dev), kernels.Workspace(dev)
    idx_h = [torch.empty((H, k), dtype=torch.int32, device=dev) for _ in range(L)]
    idx_z = [torch.empty((H, k), dtype=torch.int32, device=dev) for _ in range(L)]
    out_h = [torch.empty((N_Q, d), dtype=dtype, device=dev) for _ in range(L)]
    out_z = [torch.empty((N_Q, d), dtype=dtype, device=dev) for _ in range(L)]
    lse_h = [torch.empty((N_Q,), dtype=torch.float32, device=dev) for _ in range(L)]
    lse_z = [torch.empty((N_Q,), dtype=torch.float32, device=dev) for _ in range(L)]
    # Each layer is one call: lkv_select_hybrid_decode (bound, the top K chosen by the residency
    # launch, decode, merge) against lkv_select_decode over the same host pool.
    step_h, step_z = [], []
    for li, st in enumerate(layers):
        ss = kernels.pool_source(st["slots"])
        hs = st["hs"]
        common = dict(cand_offset=1, n_cand=n_cand, block_size=BS, scale=d**-0.5, sink=ss, sink_block=0, cur=ss, cur_block=1, fill=fill)
        step_h.append(kernels.PreparedSelectHybridDecode(q_static[li], st["kmin"], st["kmax"], k, host=hs, res=st["res"], out=out_h[li], lse=lse_h[li],
                                                         out_idx=idx_h[li], ws=ws_h, **common))
        step_z.append(kernels.PreparedSelectDecode(q_static[li], st["kmin"], st["kmax"], k, sel=hs, out=out_z[li], lse=lse_z[li], out_idx=idx_z[li],
                                                   ws=ws_z, **common))

    def capture(steps):  # noqa: ANN001, ANN202
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for f in steps:
                f()
        return g

    # Capture launches nothing; the residency tables start empty either way.
    q_static.copy_(q_seq[0])
    graph_h, graph_z = capture(step_h), capture(step_z)
    torch.cuda.synchronize()
    hist = torch.empty((S, L, H, k), dtype=torch.int32, device=dev)
    t_h, t_z = [], []
    for t in range(S):
        q_static.copy_(q_seq[t])
        e = _events(4)
        e[0].record()
        graph_h.replay()
        e[1].record()
        graph_z.replay()
        e[2].record()
        for li in range(L):
            hist[t, li].copy_(idx_h[li])
        torch.cuda.synchronize()
        t_h.append(e[0].elapsed_time(e[1]) * 1e3 / L)
        t_z.append(e[1].elapsed_time(e[2]) * 1e3 / L)
        same = all(torch.equal(out_h[li], out_z[li]) and torch.equal(lse_h[li], lse_z[li]) for li in range(L))
        assert same, f"step {t}: the hybrid output differs from the zero-copy output"
    # With k slots per head, the blocks resident at step t are step t-1's selection.
    row = (torch.arange(L * H, device=dev, dtype=torch.int64) * N).view(L, H, 1)  # make ids unique per (layer, head)
    keyed = hist.to(torch.int64) + row[None]
    hits = torch.stack([torch.isin(keyed[t], keyed[t - 1]).float().mean() for t in range(1, S)])
    hit_rate = float(hits.mean())
    warm_h = statistics.mean(t_h[1:])
    warm_z = statistics.mean(t_z[1:])
    pair = packed_pair_bytes(BS, d) if int8 else 2 * BS * d * torch.tensor([], dtype=dtype).element_size()
    miss_bytes = (1.0 - hit_rate) * H * k * pair
    log(f"hybrid128k: hybrid {warm_h:.1f} us/layer (cold step {t_h[0]:.1f}), zero-copy {warm_z:.1f} us/layer, hit rate {hit_rate:.3f}")
    step_gbps = miss_bytes / (warm_h * 1e-6) / 1e9
    roofline = {"bound": "pcie", "kernel": "the whole lkv_select_hybrid_decode call per layer (bound_kernel_mf, residency_kernel choosing the top K, "
                                            "sparse_decode_kernel reading hits from HBM slots and misses over PCIe, decode_merge_wave_kernel)",
                "achieved": round(step_gbps, 2), "peak": PCIE_PEAK_GBPS, "unit": "GB/s", "frac": round(step_gbps / PCIE_PEAK_GBPS, 4), "traffic": None,
                "algorithmic_bytes": int(miss_bytes), "step_us": round(warm_h, 2),
                "note": "the missed pairs' host bytes per layer over the warm steps' mean call time, launches and gaps included; the call is "
                        "one C entry point, so its decode launch is not timed apart here (its kernel-trace duration is in profiles/)"}
    wl = "hybrid128k_int8" if int8 else "hybrid128k"
    counted = _pmc_file().get("kernels", {}).get(f"{wl}/hybrid/sparse_decode_kernel")
    if counted:
        roofline["traffic"] = counted["traffic_bytes"]
        roofline["traffic_note"] = ("calibrated FETCH_SIZE + WRITE_SIZE bytes per hybrid decode launch: hits read from HBM slots, misses read over "
                                    f"PCIe and written into their slots; algorithmic {counted['algorithmic_bytes']} at that run's hit rate "
                                    f"{counted['hit_rate']}; source {TRAFFIC_FILE.relative_to(ROOT)}")
        roofline["traffic_run"] = pmc_run(wl, "hybrid")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_hybrid(layers, q_seq, k, n_sealed, fill, d**-0.5, args.cpu_seconds, int8, dtype, n_cand)
    return {
        "metric": "hybrid residency decode-step µs/layer over a drifting decode sequence, against the zero-copy read of the same sequence",
        "value": round(warm_h, 3), "unit": "us/layer", "n_gpus": 1, "steps": S - 1, "warmup": 1,
        "ms_per_step": round(warm_h * L / 1e3, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16" if dtype == torch.bfloat16 else "f16", "data": "synthetic",
        "config": {"workload": f"Llama-3.1-8B-shaped tiered decode, {L} layers, {T} tokens, K={k} of {n_cand} per KV head, "
                               f"{'int8 records' if int8 else 'bf16 KV'} in mapped host memory, "
                               f"{k} HBM slots per head; {S} steps whose queries are the layer's query plus N(0, {args.drift}^2 * rms^2) drift",
                   "layers": L, "tokens": T, "q_heads": N_Q, "kv_heads": H, "head_dim": d, "block_size": BS, "k": k, "drift": args.drift, "sequence_steps": S,
                   "host_tier": "int8" if int8 else "bf16"},
        "hybrid_us_per_layer": round(warm_h, 2), "hybrid_cold_step_us_per_layer": round(t_h[0], 2),
        "zerocopy_us_per_layer": round(warm_z, 2), "speedup_vs_zerocopy": round(warm_z / warm_h, 4),
        "hit_rate": round(hit_rate, 4), "pcie_bytes_per_layer": int(miss_bytes),
        "outputs_equal_zerocopy": True,
        "step_calls": "one lkv_select_hybrid_decode call per layer (bound, top K chosen in the residency launch, decode, merge: 4 launches) "
                      "against one lkv_select_decode call (bound, decode choosing the top K, merge: 3 launches)",
        "roofline": roofline,
        **({"cpu_baseline": cpu} if cpu is not None else {}),
    }


def cpu_baseline_hybrid(layers: list, q_seq, k: int, n_sealed: int, fill: int, scale: float, budget_s: float, int8: bool, dtype, n_cand: int) -> dict:  # noqa: ANN001
    """The hybrid tier's step on the CPU (oracle.cpu_path.hybrid_layer), each sampled layer stepping
    through the same drifting query sequence with its own slots and residency tables, beside the
    GPU's layer-0 output for the sequence's first query."""
    import torch

    from lazykv_amd import kernels
    from oracle import cpu_path
    from oracle.reference import residency_state

    n_layers = min(len(layers), 2)
    S = q_seq.shape[0]
    states = []
    for li in range(n_layers):
        st = layers[li]
        h, bs, d = st["kmin"].shape[1], st["slots"].shape[3], st["slots"].shape[-1]
        states.append(({"q": q_seq[:, li].cpu(), "kmin": st["kmin"].cpu(), "kmax": st["kmax"].cpu(), "host": st["host"],
                        "slots": torch.zeros((k, h, 2, bs, d), dtype=dtype), "res": residency_state(h, k, st["kmin"].shape[2]), "t": 0,
                        "sink": st["slots"][0].cpu(), "cur": st["slots"][1].cpu()},))

    def step(c: dict) -> tuple:
        t = c["t"]
        c["t"] = t + 1
        return cpu_path.hybrid_layer(c["q"][t % S], c["kmin"], c["kmax"], n_sealed, k, c["host"], c["slots"], c["res"], t, c["sink"], c["cur"], fill, scale)

    # Parity beside the timing: layer 0's first step (empty slots) against the GPU's float32 output
    # for the same query, which the hybrid call equals bit for bit (the bench asserts it per step).
    st0 = layers[0]
    ss0 = kernels.pool_source(st0["slots"])
    o32, l32 = kernels.select_decode(q_seq[0, 0], st0["kmin"], st0["kmax"], k, cand_offset=1, n_cand=n_cand, block_size=BS, scale=scale, sel=st0["hs"],
                                     sink=ss0, sink_block=0, cur=ss0, cur_block=1, fill=fill, out_dtype=torch.float32)
    torch.cuda.synchronize()
    r0 = step(states[0][0])
    parity = {"gpu_vs_cpu_layer0_max_abs_out_f32": float((r0[0] - o32.cpu()).abs().max()),
              "gpu_vs_cpu_layer0_max_abs_lse": float((r0[1] - l32.cpu()).abs().max()), "parity_bar": 2e-3}
    t = time_cpu(step, states, budget_s)
    return {
        "value": round(t["median_s"] * 1e6, 1), "unit": "us/layer", "cores": t["cores"], "kind": "port",
        "sample": f"{t['runs']} single-layer hybrid steps of layers 0-{n_layers - 1} of the same workload, each layer stepping through the "
                  f"{S}-query drifting sequence with its own {k} slots per head: fp32 quest bound, topk, admit (LRU victims, "
                  f"index_copy of the missed {'int8 records, unpacked' if int8 else 'pairs'} from the host pool into the slots), "
                  f"index_select gather from the slots, cat, masked fp32 attention + logsumexp (median over {t['runs_at_cores']} at "
                  f"{t['cores']} threads), torch CPU ops in the reference's order",
        "iqr_us": [round(x * 1e6, 1) for x in t["iqr_s"]], "per_thread_setting_us": t["per_thread_setting_us"],
        "cpu_model": cpu_model(), "host_cpus_visible": t["avail"], **parity,
    }


# -- layer-major prefill into the int8 host tier ------------------------------------------------------


def run_prefill(args: argparse.Namespace, spec: dict) -> dict:
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM

    from lazykv_amd.attention import IMPLEMENTATION_NAME, install
    from lazykv_amd.cache import FullGPUCache
    from lazykv_amd.quant import packed_pair_bytes
    from lazykv_amd.tiered import TieredCache, allocate_host_pools
    from lazykv_amd.tiered_prefill import tiered_prefill

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    n, L, d, k = spec["tokens"], spec["layers"], spec["d"], spec["k"][0]
    chunk = 4096
    reps = max(1, min(args.steps, 5))
    install()
    cfg = LlamaConfig(hidden_size=2048, intermediate_size=8192, num_hidden_layers=L, num_attention_heads=N_Q, num_key_value_heads=H, head_dim=d,
                      vocab_size=128256, max_position_embeddings=131072, rope_theta=500000.0, tie_word_embeddings=True)
    torch.manual_seed(0)
    t0 = time.time()
    with torch.device(dev):
        model = LlamaForCausalLM(cfg)  # Linear and embedding weights ~ N(0, 0.02), RMSNorm gains 1
    model.set_attn_implementation(IMPLEMENTATION_NAME)
    model = model.to(dtype=torch.float16).eval()
    gen = torch.Generator(device=dev).manual_seed(0)
    ids = torch.randint(0, cfg.vocab_size, (1, n), device=dev, generator=gen)
    cap = n + 64
    pools = allocate_host_pools(L, H, d, BS, cap, torch.float16, quant="int8")
    log(f"model and pools ready in {time.time() - t0:.1f}s")
    runs = []
    for i in range(args.warmup + reps):
        r = tiered_prefill(model, ids, chunk, k, BS, cap, dense_layers=0, host_pools=pools, quant="int8", fetch="zerocopy")
        if i >= args.warmup:
            runs.append((r.wall_s, r.boundary_layer_s, r.chunks))
        del r
    boundary_us = statistics.mean(statistics.mean(b) for _, b, _ in runs) * 1e6
    wall_s = statistics.median(w for w, _, _ in runs)
    # The path it replaces: chunk-major prefill into a full cache, then the tiers built from it.
    ref_walls = []
    for i in range(args.warmup + reps):
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        with torch.inference_mode():
            full = FullGPUCache(L, cap)
            for s in range(0, n, chunk):
                model(input_ids=ids[:, s : s + chunk], past_key_values=full, use_cache=True, logits_to_keep=1)
            cache = TieredCache(full, k, BS, cap, dense_layers=0, host_pools=pools, quant="int8", fetch="zerocopy")
        torch.cuda.synchronize()
        if i >= args.warmup:
            ref_walls.append(time.perf_counter() - w0)
        del full, cache
    ref_wall = statistics.median(ref_walls)
    nb = n // BS
    P = packed_pair_bytes(BS, d)
    # The tier build of one layer as a single launch on an otherwise idle GPU (the kernel's own
    # rate): a layer's float16 K/V in HBM -> int8 records in the mapped host pool + metadata. In the
    # prefill itself the same work is split into per-chunk launches that overlap the next chunk's
    # compute, so their summed device time (reported apart) includes the sharing.
    from lazykv_amd import kernels

    gk = torch.Generator(device=dev).manual_seed(1)
    kk = torch.randn((1, H, nb * BS, d), device=dev, generator=gk).to(torch.float16)
    vv = torch.randn((1, H, nb * BS, d), device=dev, generator=gk).to(torch.float16)
    kmin_i = torch.empty((1, H, nb, d), dtype=torch.float16, device=dev)
    kmax_i = torch.empty_like(kmin_i)
    src_i, dst_i = kernels.dense_source(kk, vv, BS), kernels.record_source(pools[0], torch.float16)

    def build_one() -> None:
        kernels.store_blocks(src_i, dst=dst_i, n_kv=H, head_dim=d, block_size=BS, first_block=0, n_blocks=nb, kmin=kmin_i, kmax=kmax_i)

    build_us = kernel_us([build_one], 5)[0]
    del kk, vv
    b_read = 2 * H * nb * BS * d * 2  # the layer's float16 K and V
    b_rec = nb * H * P  # int8 records, written to mapped host memory
    b_meta = 2 * H * nb * d * 2
    pcie = b_rec / (build_us * 1e-6) / 1e9
    pcie_in = b_rec / (boundary_us * 1e-6) / 1e9  # the same records, written by the prefill's own launches
    launches = runs[0][2]  # one store_blocks launch per chunk and selecting layer
    t_roof = max((b_read + b_meta) / (HBM_PEAK_GBPS * 1e9), b_rec / (PCIE_PEAK_GBPS * 1e9)) * 1e6
    # The link's write ceiling: the copy engines writing 512 MiB into the first layer's host pool
    # (the pool is rewritten by every later prefill, so the probe's zeros do not matter).
    write_ceiling = dma_d2h_gbps(pools[0])
    log(f"prefill32k: tier build {build_us:.1f} us/layer in one launch ({pcie:.1f} GB/s of records to host, {pcie / write_ceiling:.3f} of the copy engines' "
        f"{write_ceiling:.1f} GB/s); in the prefill, per-chunk launches overlapping "
        f"compute, {boundary_us:.1f} us/layer of device time; prefill wall {wall_s:.3f}s vs chunk-major + tier build {ref_wall:.3f}s")
    out = {
        "metric": "tiered prefill: device µs/layer of the int8 tier build inside the layer-major prefill (fused pack + key min/max, records written to "
                  "mapped host memory) & achieved PCIe GB/s (% roofline)",
        "value": round(boundary_us, 2), "unit": "us/layer", "n_gpus": 1, "steps": reps, "warmup": args.warmup,
        "ms_per_step": round(boundary_us * L / 1e3, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": f"Llama-3.2-1B-shaped layer-major prefill: {L} layers (hidden 2048, 32/8 heads, d {d}), {n}-token prompt uniform over 128,256 ids, "
                               f"float16 weights ~N(0,0.02), chunks of {chunk}, every layer's KV into the int8 host tier (dense_layers 0)",
                   "layers": L, "tokens": n, "q_heads": N_Q, "kv_heads": H, "head_dim": d, "block_size": BS, "k": k, "chunk": chunk, "dense_layers": 0,
                   "value_note": f"summed device time (events on the tier stream) of the {launches} store_blocks launches that seal each layer's blocks chunk by "
                                 "chunk while the next chunk computes; the launch shares the GPU with that compute"},
        "roofline": {"bound": "pcie", "kernel": "store_blocks_kernel (int8 records to host + metadata of the dequantised keys), one launch per chunk in the prefill",
                     "achieved": round(pcie_in, 2), "peak": PCIE_PEAK_GBPS, "unit": "GB/s", "frac": round(pcie_in / PCIE_PEAK_GBPS, 4),
                     "traffic": pmc_traffic(args.workload).get("prefill/store_blocks_kernel"),
                     "traffic_note": f"calibrated FETCH_SIZE + WRITE_SIZE bytes per launch (K/V read + records and metadata written), algorithmic per layer "
                                     f"{b_read + b_rec + b_meta}; source {TRAFFIC_FILE.relative_to(ROOT)}",
                     "algorithmic_bytes": b_rec // launches, "kernel_us": round(boundary_us / launches, 2), "launches_per_layer": launches,
                     "link_write_ceiling_gbps": round(write_ceiling, 2), "frac_of_link_write_ceiling": round(pcie_in / write_ceiling, 4)},
        "byte_roofline": {"hbm_bytes_per_layer": b_read + b_meta, "pcie_bytes_per_layer": b_rec, "t_roof_us_at_64gbps": round(t_roof, 2),
                          "frac_at_64gbps": round(t_roof / boundary_us, 4)},
        "isolated_launch": {"us_per_layer": round(build_us, 2), "pcie_gbps": round(pcie, 2), "frac_of_link_write_ceiling": round(pcie / write_ceiling, 4),
                            "hbm_read_bytes": b_read, "hbm_read_gbps": round(b_read / (build_us * 1e-6) / 1e9, 1), "metadata_bytes": b_meta,
                            "note": "one store_blocks launch over a whole layer of random K/V on an otherwise idle GPU: the kernel's own rate, not the prefill's"},
        "prefill": {"wall_s": round(wall_s, 4), "per_layer_ms": round(wall_s / L * 1e3, 3), "chunks": runs[0][2],
                    "chunk_major_then_tier_wall_s": round(ref_wall, 4), "ratio_to_chunk_major": round(wall_s / ref_wall, 4)},
    }
    if not args.no_cpu_baseline:
        from oracle import cpu_path

        with torch.inference_mode():
            full = FullGPUCache(L, cap)
            for s in range(0, n, chunk):
                model(input_ids=ids[:, s : s + chunk], past_key_values=full, use_cache=True, logits_to_keep=1)
        states = [(full.layers[i].keys[0, :, :n].cpu(), full.layers[i].values[0, :, :n].cpu(), BS) for i in range(min(2, L))]
        del full
        t = time_cpu(cpu_path.tier_build_layer, states, args.cpu_seconds)
        out["cpu_baseline"] = {
            "value": round(t["median_s"] * 1e6, 1), "unit": "us/layer", "cores": t["cores"], "kind": "port",
            "sample": f"{t['runs']} single-layer int8 tier builds of the same prefill's KV (layers 0-{len(states) - 1}): quant.py pack, unpack, key min/max in torch CPU ops "
                      f"(median over {t['runs_at_cores']} at {t['cores']} threads)",
            "iqr_us": [round(x * 1e6, 1) for x in t["iqr_s"]], "per_thread_setting_us": t["per_thread_setting_us"],
            "cpu_model": cpu_model(), "host_cpus_visible": t["avail"],
        }
    return out


if __name__ == "__main__":
    sys.exit(main())
