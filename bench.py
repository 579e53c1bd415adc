#!/usr/bin/env python3
"""Benchmark: the Llama-3.1-8B-shaped tiered decode step at 131,072 tokens and a 6.25% budget.

Workload (per decode step, 32 selecting layers): 32 query / 8 KV heads, head_dim 128, bf16 KV,
16-token blocks, 8,192 blocks per KV head of which 8,190 are candidates; K = 512 selected per KV
head. Every layer's KV lives in mapped pinned host memory (512 MiB per layer, 16 GiB in all); the
block metadata, the sink and the current block live in HBM. Per layer, one step runs the fused
Quest bound + top-K kernel over the metadata and the block-sparse decode kernel, which reads the
4,096 selected (block, head) pairs in place over PCIe. Nothing returns to the host between
layers. The 32-layer step is captured once in a HIP graph and replayed.

Reported: `value` = decode-step microseconds per layer (lower is better). Beside it: the same
step with all KV resident in HBM, per-kernel durations and their achieved bandwidth against the
byte roofline, the link probe, and the reference's CPU decode path (`oracle/cpu_path.py`) timed on
this host's cores on a bounded sample of layers.

    python bench.py [--steps K] [--warmup W] [--layers 32] [--no-cpu-baseline] [--only zerocopy|hbm]
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

METRIC = "decode-step µs/layer & achieved HBM GB/s (% roofline) at 128K ctx, 6.25% budget"
HBM_PEAK_GBPS = 8000.0
PCIE_PEAK_GBPS = 64.0  # PCIe Gen5 x16, one direction


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--layers", type=int, default=32)
    p.add_argument("--tokens", type=int, default=131072)
    p.add_argument("--k", type=int, default=512)
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--only", choices=["zerocopy", "hbm"], default=None)
    p.add_argument("--eager", action="store_true", help="launch from Python instead of replaying a graph")
    p.add_argument("--coherent", action="store_true", help="fine-grained (device-uncached) host pools")
    args = p.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path has no multi-GPU mode (asked for --gpus {args.gpus}).", file=sys.stderr)
        return 2

    import torch

    from lazykv_amd import kernels
    from lazykv_amd.pinned import device_address, pinned_empty
    from lazykv_amd.workload import draw_layer, to_pool

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    n_q, h, d, bs, k = 32, 8, 128, 16, args.k
    T, L = args.tokens, args.layers
    N = T // bs
    n_sealed, fill = N - 1, bs  # lazy sealing: the last block is the current one, full
    n_cand = n_sealed - 1
    scale = d**-0.5
    want_zc = args.only in (None, "zerocopy")
    want_hbm = args.only in (None, "hbm")

    # ---- state -------------------------------------------------------------------------------
    t0 = time.time()
    layers = []
    for li in range(L):
        w = draw_layer(li, n_q, h, d, T, bs, torch.bfloat16, device=dev)
        pool = to_pool(w.keys, w.values, bs)  # [N, h, 2, bs, d] on the GPU
        kmin = torch.zeros((1, h, N, d), dtype=torch.bfloat16, device=dev)
        kmax = torch.zeros_like(kmin)
        kernels.store_blocks(kernels.dense_source(w.keys, w.values, bs), n_kv=h, head_dim=d, block_size=bs, first_block=0, n_blocks=n_sealed, kmin=kmin, kmax=kmax)
        slots = pool[[0, N - 1]].contiguous()
        host = None
        if want_zc:
            host = pinned_empty(tuple(pool.shape), torch.bfloat16, coherent=args.coherent)
            host.copy_(pool)
        layers.append({"q": w.query.contiguous(), "kmin": kmin, "kmax": kmax, "slots": slots, "host": host, "pool": pool if want_hbm else None, "needle": w.needle})
        del w
        if not want_hbm:
            del pool
        if li % 8 == 7:
            log(f"built {li + 1}/{L} layers ({time.time() - t0:.1f}s)")
    torch.cuda.synchronize()
    log(f"state ready in {time.time() - t0:.1f}s: {L} layers x {N} blocks, host pools {'yes' if want_zc else 'no'}, HBM pools {'yes' if want_hbm else 'no'}")

    idx = torch.empty((h, k), dtype=torch.int32, device=dev)
    ws_sel, ws_dec = kernels.Workspace(dev), kernels.Workspace(dev)
    outs = [torch.empty((n_q, d), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    lses = [torch.empty((n_q,), dtype=torch.float32, device=dev) for _ in range(L)]
    ranks, decodes = [], {"zerocopy": [], "hbm": []}
    for li, st in enumerate(layers):
        ranks.append(kernels.PreparedBoundTopk(st["q"], st["kmin"], st["kmax"], k, cand_offset=1, n_cand=n_cand, out_idx=idx, ws=ws_sel))
        ss = kernels.pool_source(st["slots"])
        common = dict(n_kv=h, block_size=bs, scale=scale, idx=idx, sink=ss, sink_block=0, cur=ss, cur_block=1, fill=fill, out=outs[li], lse=lses[li], ws=ws_dec)
        if want_zc:
            decodes["zerocopy"].append(kernels.PreparedDecode(st["q"], sel=kernels.pool_source(st["host"]), **common))
        if want_hbm:
            decodes["hbm"].append(kernels.PreparedDecode(st["q"], sel=kernels.pool_source(st["pool"]), **common))

    def step(mode: str) -> None:
        for li in range(L):
            ranks[li]()
            decodes[mode][li]()

    def check(mode: str) -> None:
        """Every layer's needle is selected for every KV head; outputs are finite."""
        for li in range(L):
            ranks[li]()
            got = idx.cpu()
            needle = layers[li]["needle"]
            assert (got == needle).any(dim=1).all(), f"layer {li}: needle block {needle} not selected"
            decodes[mode][li]()
        torch.cuda.synchronize()
        assert all(torch.isfinite(o.float()).all() for o in outs), "non-finite output"

    def time_mode(mode: str) -> dict:
        check(mode)
        step(mode)
        torch.cuda.synchronize()
        graph = None
        if not args.eager:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                step(mode)
            torch.cuda.synchronize()
        run = graph.replay if graph is not None else (lambda: step(mode))
        for _ in range(args.warmup):
            run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        wall0 = time.perf_counter()
        e0.record()
        for _ in range(args.steps):
            run()
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - wall0
        ms_step = e0.elapsed_time(e1) / args.steps
        # Per-kernel durations, eager, with events on the launch stream bracketing each kernel.
        sel_ms, dec_ms = [], []
        for _ in range(max(2, min(5, args.steps))):
            for li in range(L):
                a, b, c = (torch.cuda.Event(enable_timing=True) for _ in range(3))
                a.record()
                ranks[li]()
                b.record()
                decodes[mode][li]()
                c.record()
                sel_ms.append((a, b))
                dec_ms.append((b, c))
        torch.cuda.synchronize()
        sel_us = statistics.mean(x.elapsed_time(y) for x, y in sel_ms) * 1e3
        dec_us = statistics.mean(x.elapsed_time(y) for x, y in dec_ms) * 1e3
        eager_us = None
        if graph is not None:
            torch.cuda.synchronize()
            w0 = time.perf_counter()
            for _ in range(3):
                step(mode)
            torch.cuda.synchronize()
            eager_us = (time.perf_counter() - w0) / 3 / L * 1e6
            del graph
        log(f"{mode}: {ms_step:.3f} ms/step = {ms_step * 1e3 / L:.1f} us/layer (bound+topk {sel_us:.1f} us, decode {dec_us:.1f} us), wall {wall:.2f}s")
        return {"ms_step": ms_step, "us_layer": ms_step * 1e3 / L, "sel_us": sel_us, "dec_us": dec_us, "eager_us_layer": eager_us}

    # ---- algorithmic bytes per layer (kernel-level) --------------------------------------------
    B_meta = 2 * h * n_cand * d * 2
    B_q = n_q * d * 2
    B_out = n_q * d * 2 + 4 * n_q
    B_sel = 2 * h * k * bs * d * 2
    B_sinkcur = 2 * h * 2 * bs * d * 2
    B_hbm_zc = B_meta + B_sinkcur + 2 * B_q + B_out  # q is read by both kernels

    res = {}
    if want_zc:
        res["zerocopy"] = time_mode("zerocopy")
    if want_hbm:
        res["hbm"] = time_mode("hbm")

    # ---- link and HBM probes ---------------------------------------------------------------------
    probe = {}
    sink = torch.zeros(4096, dtype=torch.int32, device=dev)

    def probe_gbps(addr: int, nbytes: int, blocks: int, reps: int = 5) -> float:
        kernels.stream_read(addr, nbytes, blocks, sink)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            kernels.stream_read(addr, nbytes, blocks, sink)
        e1.record()
        torch.cuda.synchronize()
        return nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9

    if want_zc:
        host0 = layers[0]["host"]
        probe["pcie_read_gbps"] = probe_gbps(device_address(host0), host0.numel() * 2, 2048)
    big = torch.empty(4 << 30, dtype=torch.uint8, device=dev)
    probe["hbm_read_gbps"] = probe_gbps(big.data_ptr(), big.numel(), 4096)
    del big
    log(f"probes: {probe}")

    out = {
        "metric": METRIC,
        "value": None,
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": None,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"Llama-3.1-8B-shaped tiered decode step: {L} selecting layers, {T} tokens, 16-token blocks, K={k} of {n_cand} candidates per KV head (6.25% budget), bf16 KV in mapped pinned host memory",
            "layers": L, "tokens": T, "q_heads": n_q, "kv_heads": h, "head_dim": d, "block_size": bs, "k": k,
            "rank_dtype": "float32", "dense_layers": 0, "launch": "eager" if args.eager else "hip_graph",
            "host_memory": "fine-grained" if args.coherent else "coarse-grained",
        },
        "host_syncs_per_layer": 0,
    }
    traffic = pmc_traffic()
    if want_zc:
        r = res["zerocopy"]
        pcie_gbps = B_sel / (r["dec_us"] * 1e-6) / 1e9
        t_roof64 = max((B_hbm_zc) / (HBM_PEAK_GBPS * 1e9), B_sel / (PCIE_PEAK_GBPS * 1e9)) * 1e6
        bw_probe = probe.get("pcie_read_gbps")
        t_roof_probe = max(B_hbm_zc / (HBM_PEAK_GBPS * 1e9), B_sel / (bw_probe * 1e9)) * 1e6 if bw_probe else None
        out.update(value=round(r["us_layer"], 3), ms_per_step=round(r["ms_step"], 4))
        out["roofline"] = {
            "bound": "pcie", "kernel": "lkv_sparse_decode: sparse_decode_kernel + decode_merge_kernel, zero-copy host reads", "achieved": round(pcie_gbps, 2), "peak": PCIE_PEAK_GBPS,
            "unit": "GB/s", "frac": round(pcie_gbps / PCIE_PEAK_GBPS, 4), "traffic": traffic.get("zerocopy/sparse_decode_kernel"),
            "algorithmic_bytes": B_sel, "kernel_us": round(r["dec_us"], 2),
            "traffic_note": "calibrated FETCH_SIZE + WRITE_SIZE bytes per launch, host (PCIe) and HBM fetches together; algorithmic total incl. HBM part "
            f"{B_sel + B_sinkcur + B_q + B_out}; source {TRAFFIC_FILE.relative_to(ROOT)}" if traffic else None,
        }
        out["byte_roofline"] = {
            "hbm_bytes_per_layer": B_hbm_zc, "pcie_bytes_per_layer": B_sel,
            "t_roof_us_at_64gbps": round(t_roof64, 2), "frac_at_64gbps": round(t_roof64 / r["us_layer"], 4),
            "t_roof_us_at_probe": round(t_roof_probe, 2) if t_roof_probe else None,
            "frac_at_probe": round(t_roof_probe / r["us_layer"], 4) if t_roof_probe else None,
        }
        out["kernels"] = {
            "bound_topk": {"us": round(r["sel_us"], 2), "hbm_bytes": B_meta + B_q, "gbps": round((B_meta + B_q) / (r["sel_us"] * 1e-6) / 1e9, 1),
                           "frac_hbm_peak": round((B_meta + B_q) / (r["sel_us"] * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)},
            "sparse_decode": {"us": round(r["dec_us"], 2), "pcie_bytes": B_sel, "hbm_bytes": B_sinkcur + B_q + B_out, "pcie_gbps": round(pcie_gbps, 2)},
        }
        out["eager_us_per_layer"] = round(r["eager_us_layer"], 2) if r["eager_us_layer"] else None
    if want_hbm:
        r = res["hbm"]
        b_hbm = B_meta + B_sel + B_sinkcur + 2 * B_q + B_out
        t_roof = b_hbm / (HBM_PEAK_GBPS * 1e9) * 1e6
        dec_gbps = (B_sel + B_sinkcur + B_q + B_out) / (r["dec_us"] * 1e-6) / 1e9
        sel_gbps = (B_meta + B_q) / (r["sel_us"] * 1e-6) / 1e9
        out["hbm_resident"] = {
            "us_per_layer": round(r["us_layer"], 3), "ms_per_step": round(r["ms_step"], 4), "hbm_bytes_per_layer": b_hbm,
            "t_roof_us": round(t_roof, 3), "frac": round(t_roof / r["us_layer"], 4),
            "bound_topk_us": round(r["sel_us"], 2), "bound_topk_gbps": round(sel_gbps, 1),
            "sparse_decode_us": round(r["dec_us"], 2), "sparse_decode_gbps": round(dec_gbps, 1),
            "eager_us_per_layer": round(r["eager_us_layer"], 2) if r["eager_us_layer"] else None,
        }
        if not want_zc:
            out.update(value=round(r["us_layer"], 3), ms_per_step=round(r["ms_step"], 4))
            out["config"]["workload"] = out["config"]["workload"].replace("bf16 KV in mapped pinned host memory", "bf16 KV resident in HBM")
            out["roofline"] = {"bound": "hbm", "kernel": "lkv_sparse_decode: sparse_decode_kernel + decode_merge_kernel, HBM", "achieved": round(dec_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                               "frac": round(dec_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic.get("hbm/sparse_decode_kernel"), "algorithmic_bytes": B_sel + B_sinkcur + B_q + B_out, "kernel_us": round(r["dec_us"], 2)}
    out["probes"] = {kk: round(v, 2) for kk, v in probe.items()}

    # ---- CPU baseline: the reference's decode path on this host's cores -----------------------------
    if not args.no_cpu_baseline and want_zc:
        out["cpu_baseline"] = cpu_baseline(layers, k, n_sealed, fill, scale, args.cpu_seconds, outs, lses)
    print(json.dumps(out), flush=True)
    return 0


TRAFFIC_FILE = ROOT / "profiles" / "tiered_decode_128k_pmc_traffic.json"


def pmc_traffic() -> dict:
    """Calibrated HBM/fabric bytes per launch, per "<leg>/<kernel>", from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary of this same workload (a counter run cannot time itself)."""
    try:
        with open(TRAFFIC_FILE) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return {}
    return {key: v["traffic_bytes"] for key, v in data.get("kernels", {}).items()}


def cpu_baseline(layers: list, k: int, n_sealed: int, fill: int, scale: float, budget_s: float, outs: list, lses: list) -> dict:
    import torch

    from oracle.cpu_path import decode_layer

    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cores = max(1, min(16, avail))
    settings = sorted({min(8, cores), cores})
    prev = torch.get_num_threads()
    results = {}
    n_layers = min(len(layers), 8)
    cpu_state = []
    for st in layers[:n_layers]:
        cpu_state.append((st["q"].cpu(), st["kmin"].cpu(), st["kmax"].cpu(), st["host"], st["slots"][0].cpu(), st["slots"][1].cpu()))
    # Parity sanity: the CPU path and the GPU kernels on layer 0.
    q, kmin, kmax, host, sink, cur = cpu_state[0]
    o_cpu, l_cpu, _ = decode_layer(q, kmin, kmax, n_sealed, k, host, sink, cur, fill, scale)
    gpu_diff = float((o_cpu - outs[0].float().cpu()).abs().max())
    lse_diff = float((l_cpu - lses[0].cpu()).abs().max())
    for n in settings:
        torch.set_num_threads(n)
        decode_layer(*cpu_state[0][:3], n_sealed, k, *cpu_state[0][3:], fill, scale)  # warmup
        times = []
        t_start = time.perf_counter()
        i = 0
        while (time.perf_counter() - t_start) < budget_s / len(settings) or len(times) < 3:
            q, kmin, kmax, host, sink, cur = cpu_state[i % n_layers]
            t0 = time.perf_counter()
            decode_layer(q, kmin, kmax, n_sealed, k, host, sink, cur, fill, scale)
            times.append(time.perf_counter() - t0)
            i += 1
        results[n] = times
        log(f"cpu baseline, {n} threads: median {statistics.median(times) * 1e3:.2f} ms/layer over {len(times)} layers")
    torch.set_num_threads(prev)
    best_n = cores
    med = statistics.median(results[best_n]) * 1e6
    q1, _, q3 = statistics.quantiles(results[best_n], n=4) if len(results[best_n]) >= 4 else (med, med, med)
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            cpu_model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    return {
        "value": round(med, 1), "unit": "us/layer", "cores": best_n, "kind": "port",
        "sample": f"{sum(len(v) for v in results.values())} single-layer decodes of the same workload (layers 0-{n_layers - 1}, median over {len(results[best_n])} at {best_n} threads), torch CPU ops in the reference's order: fp32 quest bound, topk, index_select gather from the host pool, cat, masked fp32 attention + logsumexp",
        "iqr_us": [round(q1 * 1e6, 1), round(q3 * 1e6, 1)] if len(results[best_n]) >= 4 else None,
        "per_thread_setting_us": {str(n): round(statistics.median(v) * 1e6, 1) for n, v in results.items()},
        "cpu_model": cpu_model, "host_cpus_visible": avail,
        "gpu_vs_cpu_layer0_max_abs_out": gpu_diff, "gpu_vs_cpu_layer0_max_abs_lse": lse_diff,
    }


if __name__ == "__main__":
    sys.exit(main())
