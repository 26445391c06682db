"""Paged GQA decode attention on one MI355X: µs per layer-step and HBM GB/s.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2] [--splits S]

A "step" is one layer-step: one paged-decode call (one kernel launch) over
one layer's KV pool for the whole batch. The workload rotates through 28
distinct layer pools (Qwen2.5-1.5B depth) so that neither L2 nor the 256 MB
MALL can serve a layer's 268 MB from cache; 28 calls are captured in one HIP
graph and the graph is replayed, timed with HIP events on the launch stream.

Configs: c1 B1x2048, c2 B16x16384 (the headline), c3
B8x32768, c3r ragged B16 with lengths ~U[512, 32768], c4 INT8 B16x16384,
c5 sparse (50% of pages, selected on the GPU each step) B8x32768, c5h the
same at B16x16384.
Inputs are synthetic N(0,1) fp16 from a seeded device generator; block
tables are a seeded permutation of the pool (non-contiguous pages).

Prints ONE JSON line. `value` is the achieved algorithmic HBM bandwidth
(bytes the path must read and write per layer-step / measured time).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
LAYERS = 28
H_KV, N_REP, D, PAGE = 2, 6, 128, 16

CONFIGS = {
    "c1": dict(batch=1, ctx=2048, kind="fp16", workload="fp16 paged decode B1 x 2048"),
    "c2": dict(batch=16, ctx=16384, kind="fp16", workload="fp16 paged decode B16 x 16384"),
    "c3": dict(batch=8, ctx=32768, kind="fp16", workload="fp16 paged decode B8 x 32768"),
    "c3r": dict(batch=16, ctx=32768, kind="fp16", ragged=True,
                workload="fp16 paged decode B16 ragged L~U[512,32768]"),
    # diagnostic: the same bytes as c2 in 512 short sequences (no split merge needed)
    "flat": dict(batch=512, ctx=512, kind="fp16", workload="fp16 paged decode B512 x 512"),
    # diagnostic: the attention shape of the full step (B16 x 8K) on its own
    "s8k": dict(batch=16, ctx=8192, kind="fp16", workload="fp16 paged decode B16 x 8192"),
    "c4": dict(batch=16, ctx=16384, kind="int8",
               workload="INT8 paged decode B16 x 16384 (fp32 scales, fp16 last-page K residual)"),
    # BASELINE configuration 5, second part: a whole decode step of the
    # Qwen2.5-1.5B geometry (28 layers, random weights) under one HIP graph.
    "step": dict(batch=16, ctx=8192, kind="step",
                 workload="full decode step, Qwen2.5-1.5B geometry (28 layers, hidden 1536, "
                          "vocab 151936, random init), B16 x 8K, HIP graph bucket 8192"),
    "c5": dict(batch=8, ctx=32768, kind="sparse", ratio=0.5,
               workload="sparse 50% paged decode B8 x 32768 (page index + top-k + page-subset "
                        "attention)"),
    # the sparse variant at the headline shape
    "c5h": dict(batch=16, ctx=16384, kind="sparse", ratio=0.5,
                workload="sparse 50% paged decode B16 x 16384 (page index + top-k + page-subset "
                         "attention)"),
}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2800)
    p.add_argument("--warmup", type=int, default=280)
    p.add_argument("--config", default=None, choices=sorted(CONFIGS),
                   help="one configuration (default: c2, with the other attention "
                        "configurations timed after it unless --no-others)")
    p.add_argument("--splits", type=int, default=None)
    p.add_argument("--layers", type=int, default=LAYERS)
    p.add_argument("--tables", default="random", choices=["random", "contiguous"],
                   help="block-table layout (contiguous: the pages of a sequence are adjacent, "
                        "a diagnostic of the gather's cost)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-others", action="store_true",
                   help="the default run: skip timing the other attention configurations "
                        "(reported under 'other_configs' of the same line)")
    p.add_argument("--cpu-seqs", type=int, default=None,
                   help="sequences in the CPU-baseline sample (default: the whole batch)")
    p.add_argument("--compute-probe", type=int, default=0, metavar="ITEMS",
                   help="instead of the benchmark, time the decode kernel's page compute alone "
                        "(MFMA, as built) against a VALU formulation, ITEMS pages a wave, from "
                        "the measurement build given by --diag-lib, and exit")
    p.add_argument("--timeline", default=None, metavar="PATH",
                   help="instead of the benchmark, run the config's layer launches from the "
                        "-DLS_STAMPS build at PATH (python -m latentserve_amd.csrc.build "
                        "--stamps PATH) and print where each launch's time goes, from every "
                        "workgroup's clock stamps, then exit")
    p.add_argument("--diag-lib", default=None, metavar="PATH",
                   help="the -DLS_DIAGNOSTICS build (python -m latentserve_amd.csrc.build "
                        "--diagnostics PATH) that holds the page-compute probe")
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                   help="instead of the benchmark, run device copies of MIB MiB (for the "
                        "rocprof FETCH_SIZE / WRITE_SIZE scale factor) and exit")
    return p.parse_args()


def lengths_for(cfg, gen_seed=1234):
    import numpy as np
    b = cfg["batch"]
    if cfg.get("ragged"):
        rng = np.random.default_rng(gen_seed)
        return rng.integers(512, cfg["ctx"] + 1, size=b).astype(np.int32)
    return np.full(b, cfg["ctx"], np.int32)


def algorithmic_bytes(cfg, lens) -> int:
    """Bytes one layer-step must move: the live K/V (and INT8 scales and
    residual), q, the live block-table entries, lengths, and the output."""
    pages = [(int(l) + PAGE - 1) // PAGE for l in lens]
    tokens = sum(p * PAGE for p in pages)          # whole pages are read
    b = len(lens)
    if cfg["kind"] == "sparse":
        # indexer: kmin + kmax of every scored page; attention: the kept pages
        ratio = cfg["ratio"]
        width = (cfg["ctx"] + PAGE - 1) // PAGE
        k = min(width, max(3, math.ceil(ratio * width)))
        scored = sum(max(0, p - 3) for p in pages)
        kept = sum(min(k, p, max(3, math.ceil(ratio * p))) for p in pages)
        bounds = scored * H_KV * D * 2 * 2
        kv = kept * PAGE * H_KV * D * 2 * 2
        q = b * H_KV * N_REP * D * 2
        sel = b * H_KV * k * 4
        return bounds + kv + 2 * q + sum(pages) * 4 + kept * H_KV * 4 + sel + b * 4
    if cfg["kind"] == "fp16":
        kv = tokens * H_KV * D * 2 * 2
    else:
        full_pages = sum(max(0, p - 1) for p in pages)
        kv = (tokens * H_KV * D * 1 * 2                    # int8 K and V codes
              + full_pages * H_KV * D * 4                  # K scale per (block, head, ch)
              + tokens * H_KV * 4                          # V scale per (block, tok, head)
              + b * PAGE * H_KV * D * 2)                   # last page of K from the residual
    q = b * H_KV * N_REP * D * 2
    out = q
    tables = sum(pages) * 4 + b * 4
    return kv + q + out + tables


def build_workload(cfg, layers, seed=0, contiguous=False):
    import numpy as np
    import torch

    dev = torch.device("cuda", 0)
    lens = lengths_for(cfg)
    b = cfg["batch"]
    max_pages = max(1, (int(lens.max()) + PAGE - 1) // PAGE)
    width = (cfg["ctx"] + PAGE - 1) // PAGE
    nb = b * width + 4
    g = torch.Generator(device=dev).manual_seed(seed)
    if contiguous:
        tables = torch.arange(b * width, device=dev).view(b, width)
    else:
        tables = torch.randperm(nb, device=dev, generator=g)[: b * width].view(b, width)
    tables = tables.to(torch.int32).contiguous()
    seq = torch.from_numpy(lens).to(dev)
    pools = []
    for _ in range(layers):
        q = torch.randn(b, H_KV, N_REP, D, device=dev, generator=g, dtype=torch.float16)
        k = torch.randn(nb, PAGE, H_KV, D, device=dev, generator=g, dtype=torch.float16)
        v = torch.randn(nb, PAGE, H_KV, D, device=dev, generator=g, dtype=torch.float16)
        if cfg["kind"] == "int8":
            pools.append((q,) + quantize_layer(k, v, tables, seq))
        elif cfg["kind"] == "sparse":
            from latentserve_amd.kernels.hip import paged_sparse as ps
            kmin = torch.empty(nb, H_KV, D, dtype=torch.float16, device=dev)
            kmax = torch.empty_like(kmin)
            ps.rebuild_bounds(k, kmin, kmax)
            pools.append((q, k, v, kmin, kmax))
        else:
            pools.append((q, k, v))
    return tables, seq, pools, int(max_pages * PAGE)


def quantize_layer(k, v, tables, seq):
    """INT8 pools from fp16 N(0,1) data with the reference's symmetric scheme
    (cache/int8_paged_cache.py:670-699 for K per (block, head, channel),
    :741-758 for V per (block, token, head)); every sequence's last page of K
    also stays in an fp16 residual, as the cache's invariant holds
    (:283-298). Benchmark input set-up only (torch ops; not timed)."""
    import torch

    f = k.float()
    ks = f.abs().amax(dim=1).clamp_min(1e-8) / 127
    kq = torch.clamp(torch.round(f / ks.unsqueeze(1)), -127, 127).to(torch.int8)
    del f
    vf = v.float()
    vs = vf.abs().amax(dim=-1).clamp_min(1e-8) / 127
    vq = torch.clamp(torch.round(vf / vs.unsqueeze(-1)), -127, 127).to(torch.int8)
    del vf
    b = tables.shape[0]
    last = ((seq.long() + PAGE - 1) // PAGE - 1).clamp(min=0)
    res = k[tables[torch.arange(b, device=k.device), last].long()].contiguous()
    res_rows = torch.arange(b, dtype=torch.int32, device=k.device)
    return kq, vq, ks.contiguous(), vs.contiguous(), res, res_rows


def make_call(cfg, tables, seq, layer, max_len, splits):
    from latentserve_amd.kernels.hip import paged_decode_hip as pdh

    if cfg["kind"] == "int8":
        q, kq, vq, ks, vs, res, rr = layer
        return lambda: pdh.paged_decode_hip(q, kq, vq, tables, seq, max_len, num_splits=splits,
                                            k_scale=ks, v_scale=vs, k_residual=res, res_rows=rr)
    if cfg["kind"] == "sparse":
        from latentserve_amd.kernels.hip import paged_sparse as ps
        q, k, v, kmin, kmax = layer
        return lambda: ps.sparse_attention(q, k, v, tables, seq, kmin, kmax, ratio=cfg["ratio"],
                                           max_seq_len=max_len)
    q, k, v = layer
    return lambda: pdh.paged_decode_hip(q, k, v, tables, seq, max_len, num_splits=splits)


def cpu_baseline(cfg, tables, seq, layer, n_seqs):
    """The CPU oracle (a C restatement of the reference's paged_decode_reference
    loop) over a sample of the same workload, on this host's cores."""
    import numpy as np

    import oracle

    threads = min(host_cores(), 16)
    oracle.set_num_threads(threads)
    b = cfg["batch"]
    n = min(b, n_seqs or b)
    lens = seq.cpu().numpy()[:n]
    t = tables.cpu().numpy()[:n]
    if cfg["kind"] == "sparse":
        q, k, v, kmin, kmax = [x.cpu().numpy() for x in layer]
        width = t.shape[1]
        kk = oracle.budget(cfg["ratio"], width)
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            scores = oracle.page_scores(q[:n], kmin, kmax, t, lens)
            sel = oracle.select(scores, kk)
            oracle.sparse_decode(q[:n], k, v, t, lens, sel, ratio=cfg["ratio"])
            times.append(time.perf_counter() - t0)
        return _cpu_result(cfg, lens, b, n, sorted(times)[1], threads,
                           "C oracle page_scores + stable top-k + sparse_decode")
    if cfg["kind"] == "int8":
        q, kq, vq, ks, vs, res_k, rr = [x.cpu().numpy() for x in layer]
        args = (q[:n], kq, vq, t, lens)
        extra = dict(k_scale=ks, v_scale=vs, k_residual=res_k, res_rows=rr[:n])
    else:
        q, k, v = [x.cpu().numpy() for x in layer]
        args = (q[:n], k, v, t, lens)
        extra = {}
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        oracle.paged_decode(*args, num_splits=1, **extra)
        times.append(time.perf_counter() - t0)
    res = _cpu_result(cfg, lens, b, n, sorted(times)[1], threads,
                      "C oracle paged_decode (num_splits=1)")
    if cfg["kind"] == "fp16":
        res["vectorised"] = cpu_gather_sdpa(q[:n], k, v, t, lens, b, threads, cfg)
    else:
        res["vectorised"] = cpu_gather_sdpa(q[:n], kq, vq, t, lens, b, threads, cfg,
                                            int8=(ks, vs, res_k, rr[:n]))
    return res


def cpu_gather_sdpa(q, k, v, tables, lens, b, threads, cfg, int8=None):
    """The second CPU line: the reference's CPU gather path (each sequence's
    pages gathered into contiguous K/V, dequantized for an INT8 pool with the
    last page of K from the fp16 residual, then one fp32 attention of the
    n_rep query rows of each KV head over them; model/attention/gqa.py:
    351-388, cache/paged_cache.py:486-506, kernels/gqa/paged_decode.py:
    122-148), in torch on the same sample."""
    import torch

    torch.set_num_threads(threads)
    kt, vt = torch.from_numpy(k), torch.from_numpy(v)
    qt = torch.from_numpy(q).float()
    n, h, r, d = qt.shape
    page = kt.shape[1]
    scale = 1.0 / math.sqrt(d)
    if int8 is not None:
        kst, vst, krt = (torch.from_numpy(x) for x in int8[:3])
        rows = int8[3]

    def gather(i, L):
        np_ = -(-L // page)
        idx = torch.from_numpy(tables[i, :np_].astype("int64"))
        if int8 is None:
            kk = kt[idx].float()
            vv = vt[idx].float()
        else:
            kk = kt[idx].float() * kst[idx][:, None]                       # [P, 16, h, d]
            vv = vt[idx].float() * vst[idx][..., None]
            kk[np_ - 1] = krt[int(rows[i])].float()                        # the residual page
        return (kk.reshape(-1, h, d)[:L].transpose(0, 1),                 # [h, L, d]
                vv.reshape(-1, h, d)[:L].transpose(0, 1))

    def run():
        for i in range(n):
            kk, vv = gather(i, int(lens[i]))
            torch.nn.functional.scaled_dot_product_attention(qt[i], kk, vv, scale=scale)

    run()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    dt = sorted(times)[1]
    sample_bytes = algorithmic_bytes(cfg, lens)
    return {"value": round(sample_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
            "ms_per_layer_step": round(dt * 1e3 * b / n, 3),
            "sample": f"{n} of {b} sequences, torch CPU gather"
                      f"{' + dequant' if int8 is not None else ''} + fp32 SDPA of the n_rep rows "
                      f"of each KV head, median of 3 (after one untimed run)"}


def host_cores() -> int:
    """CPUs this process may run on (the box's share), else the machine's count."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def _cpu_result(cfg, lens, b, n, dt, threads, what):
    sample_bytes = algorithmic_bytes(cfg, lens)
    return {
        "value": round(sample_bytes / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "host_cores": host_cores(),
        "kind": "port",
        "sample": f"{n} of {b} sequences of one layer-step ({sample_bytes / 1e6:.1f} MB), "
                  f"{what} (oracle/ls_oracle.c, OpenMP), median of 3: "
                  f"{dt * 1e3:.1f} ms -> {dt * 1e3 * b / n:.1f} ms per full layer-step",
        "ms_per_layer_step": round(dt * 1e3 * b / n, 3),
    }


def calibrate_copy(mib):
    import torch
    n = mib * (1 << 20)
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    src.fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": n, "launches": 5}))


def compute_probe(items, diag_lib):
    """The page compute from registers, 8 waves a CU as the decode kernel
    runs: one page's QK, softmax and PV per wave, MFMA (mode 0) against VALU
    (mode 1), from the measurement build's ls_compute_probe.  Every wave
    applies one synthetic page (16 tokens, 6 rows, 128 channels, values
    exact in fp16) `items` times, so its output equals the page's fp32
    attention whatever `items` is."""
    import ctypes

    import torch
    if not diag_lib:
        sys.exit("--compute-probe needs --diag-lib PATH (the -DLS_DIAGNOSTICS build)")
    lib = ctypes.CDLL(diag_lib)
    fn = lib.ls_compute_probe
    fn.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_void_p,
                   ctypes.c_void_p]
    t = torch.arange(16).view(-1, 1)
    r = torch.arange(6).view(-1, 1)
    ch = torch.arange(128).view(1, -1)
    k = ((t * 7 + ch * 3) % 17 - 8).float() * 0.0625
    v = ((t * 5 + ch * 11) % 13 - 6).float() * 0.125
    q = ((r * 13 + ch * 5) % 11 - 5).float() * 0.125
    scale = 1.0 / math.sqrt(128)
    want = (torch.softmax((q @ k.t()) * scale, dim=-1) @ v).cuda()
    stream = torch.cuda.current_stream().cuda_stream
    res = {"items_per_wave": items}
    for groups in (256, 512):
        for mode, name in ((0, "mfma"), (1, "valu")):
            out = torch.empty(groups * 8, 6, 128, dtype=torch.float32, device="cuda")
            assert fn(mode, groups, 8, scale, out.data_ptr(), stream) == 0
            torch.cuda.synchronize()
            err = (out - want).abs().max().item()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(5):
                assert fn(mode, groups, items, scale, out.data_ptr(), stream) == 0
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / 5
            res[f"{name}_g{groups}"] = {"us": round(us, 2),
                                        "ns_per_page_per_wave": round(us * 1e3 / items, 2),
                                        "max_abs_err": err}
    print(json.dumps(res))


# The decode's stamp points (csrc/ls_decode.hip, ls_select.h; LS_STAMP).
STAMP_NAMES = {0: "group start", 1: "own share scored", 2: "scores released, counted",
               3: "peers' count seen", 4: "row keys requested", 13: "extrema barrier",
               14: "histogram barrier", 5: "threshold search done", 6: "list emitted",
               7: "walk start", 8: "wave 0 walk end", 9: "waves merged, records stored",
               10: "records released", 11: "arrival counted", 12: "combine done"}


def timeline(cfg, args):
    """Where one launch's time goes: every workgroup's stamps (100 MHz clock)
    relative to the launch's first group start, median and spread over the
    groups of several launches (the last of 8 layer launches each time, so
    its pools are cold in L2 and MALL)."""
    import ctypes

    import numpy as np
    import torch
    os.environ["LATENTSERVE_HIP_LIB"] = os.path.abspath(args.timeline)
    tables, seq, pools, max_len = build_workload(cfg, 8)
    calls = [make_call(cfg, tables, seq, lay, max_len, args.splits) for lay in pools]
    for _ in range(20):
        for c in calls:
            c()
    torch.cuda.synchronize()
    lib = ctypes.CDLL(os.environ["LATENTSERVE_HIP_LIB"])
    buf = np.zeros(8192 * 32, np.uint64)
    rel, xcd_ok, groups = [], 0, 0
    spread = {"launch_end": [], "max_minus_median": [], "xcd_median_range": [],
              "within_xcd_range_median": []}
    for _ in range(8):
        for c in calls:
            c()
        torch.cuda.synchronize()
        assert lib.ls_diag_read_stamps(buf.ctypes.data_as(ctypes.c_void_p),
                                       ctypes.c_size_t(buf.nbytes)) == 0
        st = buf.reshape(8192, 32).astype(np.int64)
        t0 = st[:, 0]
        last = np.where(t0 > t0.max() - 10000)[0]          # the last launch's groups
        base = st[last, 0].min()
        s = st[last, :15]
        rel.append(np.where(s >= base, (s - base) * 0.01, np.nan))
        xcd_ok += int(((last % 8) == (st[last, 15] & 15)).sum())
        groups += len(last)
        # where the groups' merge times spread: between XCDs or within one
        merged = (st[last, 9] - base) * 0.01
        xcd = st[last, 15] & 15
        ok = st[last, 9] >= base
        if ok.any():
            m, x = merged[ok], xcd[ok]
            meds = [float(np.median(m[x == k])) for k in range(8) if (x == k).any()]
            rngs = [float(np.ptp(m[x == k])) for k in range(8) if (x == k).sum() > 1]
            spread["launch_end"].append(float(m.max()))
            spread["max_minus_median"].append(float(m.max() - np.median(m)))
            spread["xcd_median_range"].append(max(meds) - min(meds))
            spread["within_xcd_range_median"].append(float(np.median(rngs)) if rngs else 0.0)
            spread.setdefault("xcd_medians", []).append(
                [round(float(np.median(m[x == k])), 1) if (x == k).any() else None
                 for k in range(8)])
    rel = np.concatenate(rel)
    out = {"config": cfg["workload"], "launches": 8, "groups": groups,
           "groups_on_xcd_L_mod_8": xcd_ok, "us_from_first_group_start": {},
           "merge_spread_us (median over launches)": {
               k: round(float(np.median(v)), 2) for k, v in spread.items()
               if v and k != "xcd_medians"},
           "xcd_median_merge_us_per_launch": spread.get("xcd_medians", [])}
    order = ([0, 1, 2, 3, 4, 13, 14, 5, 6, 7, 8, 9, 10, 11, 12] if cfg["kind"] == "sparse"
             else [0, 8, 1, 2, 9, 10, 11, 12])
    for i in order:
        col = rel[:, i]
        col = col[~np.isnan(col)]
        if len(col):
            name = STAMP_NAMES[i]
            if cfg["kind"] != "sparse" and i in (1, 2):
                name = {1: "first wave's walk end", 2: "last wave's walk end"}[i]
            out["us_from_first_group_start"][name] = {
                "groups": int(len(col)), "p10": round(float(np.percentile(col, 10)), 2),
                "median": round(float(np.median(col)), 2),
                "p90": round(float(np.percentile(col, 90)), 2), "max": round(float(col.max()), 2)}
    print(json.dumps(out, indent=1))


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU (got --gpus {args.gpus}); the decode path "
              "shards by sequence with no exchange, so N GPUs = N x one GPU's number",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
    if args.compute_probe:
        compute_probe(args.compute_probe, args.diag_lib)
        return
    default_run = args.config is None
    args.config = args.config or "c2"
    cfg = CONFIGS[args.config]
    if args.timeline:
        return timeline(cfg, args)
    if cfg["kind"] == "step":
        return bench_step(cfg, args)
    tables, seq, pools, max_len, splits, nbytes, ms_step = measure(cfg, args)
    gbps = nbytes / (ms_step * 1e-3) / 1e9
    layers = max(1, args.layers)

    result = {
        "metric": "paged-decode attn us/layer-step + HBM GB/s (% of 8 TB/s peak), B16x16K fp16",
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "us_per_layer_step": round(ms_step * 1e3, 3),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 KV / fp16 q" if cfg["kind"] == "int8" else "fp16",
        "data": "synthetic N(0,1), seeded device generator, permuted block tables",
        "config": {"workload": cfg["workload"], "batch": cfg["batch"], "ctx": cfg["ctx"],
                   "kv_heads": H_KV, "n_rep": N_REP, "head_dim": D, "page": PAGE,
                   "layer_pools": layers, "num_splits": splits,
                   "algorithmic_bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                     "traffic": traffic_from_profiles(args.config)},
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(cfg, tables, seq, pools[0], args.cpu_seqs)
    if default_run and not args.no_others and args.splits is None:
        del tables, seq, pools
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        result["other_configs"] = other_configs(args)
    print(json.dumps(result))


def measure(cfg, args, splits=None):
    """The layer-step time of one attention configuration: its workload on
    `args.layers` pools, a graph of `args.steps` launches replayed after
    `args.warmup` eager ones, HIP events around the replays."""
    import torch

    layers = max(1, args.layers)
    tables, seq, pools, max_len = build_workload(cfg, layers, contiguous=args.tables == "contiguous")
    lens = seq.cpu().numpy()
    nbytes = algorithmic_bytes(cfg, lens)
    from latentserve_amd.kernels.hip import paged_decode_hip as pdh
    splits = splits or args.splits or pdh.choose_splits(cfg["batch"], H_KV, (max_len + PAGE - 1) // PAGE,
                                              torch.device("cuda", 0),
                                              int8=cfg["kind"] == "int8")
    calls = [make_call(cfg, tables, seq, pools[i], max_len, splits) for i in range(layers)]

    for i in range(args.warmup):
        calls[i % layers]()
    torch.cuda.synchronize()

    def capture(n):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                calls[i % layers]()
        return g

    full, rem = divmod(args.steps, layers)
    g_full = capture(layers) if full else None
    g_rem = capture(rem) if rem else None
    # every graph is replayed once before the timed region (its first replay
    # uploads it), so the timed replays measure the kernels alone
    for g in (g_full, g_rem):
        if g is not None:
            g.replay()
    torch.cuda.synchronize()

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(full):
        g_full.replay()
    if g_rem is not None:
        g_rem.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    ms_step = ms / args.steps
    return tables, seq, pools, max_len, splits, nbytes, ms_step



def other_configs(args):
    """The other attention configurations of the configuration table, each
    measured as the headline is (same steps, warm-up and layer pools) in a
    process of its own (`bench.py --config X --no-cpu`, a child process):
    timed in this process after the headline's pools were freed, the same
    launches ran 2-5 % slower (c3 49.6 against 47.2 us alone).  A
    configuration that fails is reported with its error and does not stop
    the run."""
    import subprocess
    out = {}
    for name in ("c1", "c3", "c3r", "c4", "c5", "c5h", "s8k"):
        cmd = [sys.executable, os.path.abspath(__file__), "--config", name, "--no-cpu",
               "--steps", str(args.steps), "--warmup", str(args.warmup),
               "--layers", str(args.layers)]
        try:
            p = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
            lines = [ln for ln in p.stdout.strip().splitlines() if ln.startswith("{")]
            if p.returncode != 0 or not lines:
                out[name] = {"error": f"exit {p.returncode}: {p.stderr.strip()[-300:]}"}
                continue
            r = json.loads(lines[-1])
            out[name] = {"workload": r["config"]["workload"],
                         "us_per_layer_step": r["us_per_layer_step"],
                         "algorithmic_gbps": r["value"], "hbm_frac": r["hbm_frac"],
                         "num_splits": r["config"]["num_splits"],
                         "algorithmic_bytes_per_step": r["config"]["algorithmic_bytes_per_step"]}
        except Exception as e:   # reported, not raised: the headline line still prints
            out[name] = {"error": f"{type(e).__name__}: {e}"}
    return out


def bench_step(cfg, args):
    """Whole decode steps through the graph runner: every step is the cache's
    host bookkeeping, one graph replay (28 layers: GEMMs, RoPE, the K/V write,
    the HIP paged decode) and the greedy argmax, for B sequences at ~ctx."""
    import torch

    from latentserve_amd.runtime.hip_graph import GraphedDecoder
    from latentserve_amd.runtime.qwen_decoder import DecoderConfig, QwenDecoder

    b, ctx = cfg["batch"], cfg["ctx"]
    steps = min(args.steps, 150)
    warm = min(args.warmup, 20)
    start = ctx - steps - warm - 2                 # every timed step stays in the one bucket
    model = QwenDecoder(DecoderConfig())
    cache = model.allocate_cache(b, ctx)
    cache.advance(start, batch_size=b)             # the context's slots, filled directly:
    g = torch.Generator(device="cuda").manual_seed(1)
    for layer in range(model.cfg.num_layers):      # K/V of a `start`-token context
        cache.k_pool[layer].normal_(generator=g)
        cache.v_pool[layer].normal_(generator=g)
    dec = GraphedDecoder(model, buckets=(ctx,), greedy=True)
    tok = torch.randint(0, model.cfg.vocab_size, (b, 1), device="cuda", generator=g)
    slots = list(range(b))

    def one(t):
        pos = torch.full((b, 1), start + t, dtype=torch.long, device="cuda")
        return dec.step_greedy(tok, pos, slots)

    for t in range(warm + 1):
        nxt = one(t)
        tok.copy_(nxt)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(warm + 1, warm + 1 + steps):
        nxt = one(t)
        tok.copy_(nxt)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    st = dec.stats()
    result = {
        "metric": "full decode step tokens/s (B16 x 8K, Qwen2.5-1.5B geometry)",
        "value": round(b / dt, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: random-init weights, N(0,1) K/V context, greedy tokens",
        "config": {"workload": cfg["workload"], "batch": b, "context_start": start,
                   "layers": model.cfg.num_layers, "graphs": st["graphs"],
                   "graph_steps": st["graph_steps"], "eager_steps": st["eager_steps"],
                   "host_ms_last_step": round(dec.last_host_ms, 3)},
    }
    print(json.dumps(result))


def traffic_from_profiles(config):
    """HBM bytes per launch from the committed rocprofv3 counter summary
    (profiles/traffic_<config>.json: FETCH_SIZE + WRITE_SIZE per dispatch,
    scaled by a plain copy's counter-to-bytes factor), or None."""
    path = os.path.join(ROOT, "profiles", f"traffic_{config}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


if __name__ == "__main__":
    main()
