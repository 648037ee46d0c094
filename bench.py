"""Paged GQA decode benchmark on one MI355X.

One step = one ``attention_amd.gqa_decode`` call over the whole batch of the
workload (default cfg2, the Qwen3-8B-shaped config BASELINE.json's target is
quoted on), with q/K/V/metadata already resident in HBM.  The timed region
rotates over several K/V pools whose total exceeds the 256 MB Infinity Cache
so that every call streams its K/V from HBM.  Output allocation is inside
the timed region, as in the reference's measurement
(reference ``benchmarks/measure_decode.py:40``).

Prints one JSON line: ``value`` is achieved algorithmic HBM GB/s per call
(bytes = K+V of valid tokens + q + out + lengths + used table entries),
``us_per_call`` the latency; ``roofline`` the decode kernel's fraction of
the 8 TB/s HBM peak; ``cpu_baseline`` the reference CPU path timed on the
host cores.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg2]
  python bench.py --mode copy     # HBM copy of known size (counter calibration)
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import torch  # noqa: E402

PEAK_HBM_GBS = 8000.0
METRIC = "paged GQA decode µs/call and achieved HBM GB/s (% of peak), 1 MI355X"
DT_NAME = {torch.float32: "fp32", torch.float16: "fp16", torch.bfloat16: "bf16"}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="cfg2")
    ap.add_argument("--pools", type=int, default=0, help="K/V pools to rotate (0: enough for >768 MB)")
    ap.add_argument("--kernel", choices=["auto", "generic"], default="auto",
                    help="generic: force the portable VALU kernel through the C ABI")
    ap.add_argument("--splits", type=int, default=0, help="override the plan (C ABI path)")
    ap.add_argument("--chunk-pages", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-repeats", type=int, default=5)
    ap.add_argument("--mode", choices=["decode", "copy", "stamps", "read"], default="decode",
                    help="copy: HBM copy of known size (counter calibration); stamps: per-wave timestamps "
                         "of the balanced decode kernel (with --op mla: of the MLA shared-tile attention "
                         "kernel on --mla-config); read: streaming-read ceiling of the decode access "
                         "pattern (both from the diagnostic library)")
    ap.add_argument("--merge", choices=["auto", "fused", "unfused"], default="auto",
                    help="where split sequences are merged (C ABI path, QD_STAGE_FUSED/UNFUSED)")
    ap.add_argument("--launches", type=int, default=6, help="--mode stamps: launches recorded")
    ap.add_argument("--probe-pf", type=int, default=2, help="--mode read: groups in flight per wave (1-4)")
    ap.add_argument("--probe-split", type=int, default=1, choices=(1, 2),
                    help="--mode read: sets of waves taking alternate groups (2: twice the waves per CU)")
    ap.add_argument("--probe-work", type=int, default=0,
                    help="--mode read: dependent multiply-adds per group standing in for the decode math")
    ap.add_argument("--op", choices=["decode", "kv_append", "mla", "sweep", "splits", "models"], default="decode",
                    help="kv_append: time the paged cache append on the config's shapes instead; "
                         "mla: time paged MLA decode (attention_amd.mla_decode) on --mla-config; "
                         "sweep: the reference's decode sweep (benchmarks/measure_decode.py:43-57); "
                         "splits: the split layout by split count on the sweep's fp32 shapes; "
                         "models: the automatic path on common model shapes (MODEL_SHAPES)")
    ap.add_argument("--model", default="", help="--op models: one shape of MODEL_SHAPES, in this process")
    ap.add_argument("--mla-config", default="mla-h128")
    ap.add_argument("--mla-kernel", choices=["auto", "wave", "staged"], default="auto",
                    help="--op mla: attention kernel of the timed attention stage (comparison)")
    ap.add_argument("--device-gen", action="store_true", help="draw inputs on the GPU")
    ap.add_argument("--compute", choices=["mfma", "valu"], default="mfma",
                    help="valu: the balanced kernel with VALU math in place of MFMA (QD_STAGE_VALU, "
                         "C ABI path), for the MFMA-versus-VALU comparison")
    return ap.parse_args()


def time_loop(fn, steps: int, warmup: int, stream) -> float:
    """Milliseconds per step: HIP events on `stream` around exactly `steps` calls."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


SAMPLES = 5


def time_samples(fn, steps: int, warmup: int, stream, samples: int = SAMPLES) -> list[float]:
    """The reference's timing method (benchmarks/measure_decode.py:47-57):
    `warmup` untimed calls, then `samples` samples of exactly `steps` calls,
    each bracketed by synchronizations and HIP events on `stream`.
    Milliseconds per call of each sample; callers report the median."""
    for i in range(warmup):
        fn(i)
    out = []
    for s in range(samples):
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(steps):
            fn(s * steps + i)
        end.record(stream)
        torch.cuda.synchronize()
        out.append(start.elapsed_time(end) / steps)
    return out


def graph_replay_us(enqueue, stream, calls: int = 10, reps: int = 10) -> float:
    """GPU time per call without host overhead: `calls` calls of `enqueue`
    (which must allocate nothing and enqueue no memset) captured in one HIP
    graph, replayed `reps` times per sample between HIP events; median of
    SAMPLES samples, microseconds per call."""
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        for _ in range(3):
            enqueue()
    stream.wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            enqueue()
    graph.replay()
    torch.cuda.synchronize()
    out = []
    for _ in range(SAMPLES):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps):
            graph.replay()
        end.record(stream)
        torch.cuda.synchronize()
        out.append(start.elapsed_time(end) / (reps * calls) * 1e3)
    del graph
    return statistics.median(out)


def copy_mode(args) -> None:
    n = 1 << 30  # bytes per copy
    src = torch.empty(n, dtype=torch.uint8, device="cuda").random_()
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream()
    ms = time_loop(lambda i: dst.copy_(src), args.steps, args.warmup, stream)
    gbs = 2 * n / (ms * 1e-3) / 1e9
    print(json.dumps({"mode": "copy", "bytes_read_per_call": n, "bytes_written_per_call": n,
                      "ms_per_call": ms, "gbs": gbs}), flush=True)


def _pct(xs, q):
    xs = sorted(xs)
    return xs[min(len(xs) - 1, max(0, int(round(q * (len(xs) - 1)))))]


def stamps_mode(args) -> None:
    """Per-wave s_memrealtime stamps (100 MHz) of the balanced decode kernel,
    from attention_amd/lib/libqd_attention_diag.so (gqa_decode.hip built
    with -DQD_STAMPS): entry, end of the partition search, end of streaming,
    partial stores retired, arrival atomics returned, last merge done (the
    last three for the fused merge), and the XCD.  --launches launches, each
    alone on an idle GPU, over rotated K/V pools; one JSON line per launch
    with the phase times in microseconds from the first wave's entry."""
    import ctypes
    from attention_amd import _build, cabi
    from attention_amd.cases import get_config

    L = ctypes.CDLL(_build.DIAG_LIB)
    V, I, I64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
    L.qd_diag_set_stamps.argtypes = [V]
    L.qd_gqa_decode_auto_stages.argtypes = [V] * 7 + [ctypes.c_size_t] + [I] * 6 + [I64, I, F, I, V]
    L.qd_gqa_decode_auto_info.argtypes = [I] * 7 + [ctypes.POINTER(I)] * 3
    L.qd_error_string.restype = ctypes.c_char_p
    cfg = get_config(args.config)
    dev = torch.device("cuda:0")
    lengths = cfg.lengths()
    case = (cfg.make(device=dev, device_gen=True, lengths=lengths) if args.device_gen
            else tuple(x.to(dev) for x in cfg.make(device="cpu", lengths=lengths)))
    q, k, v, table, lens = case
    kv_bytes = 2 * k.numel() * k.element_size()
    pools = args.pools or max(2, math.ceil(768e6 / kv_bytes))
    ks, vs = [k], [v]
    for i in range(1, pools):
        ks.append(k.roll(i, dims=0).contiguous())
        vs.append(v.roll(i, dims=0).contiguous())
    dt = cabi.DTYPE[q.dtype]
    w_, s_, c_ = I(), I(), I()
    kind = L.qd_gqa_decode_auto_info(cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.block_size,
                                     table.shape[1], dt, ctypes.byref(w_), ctypes.byref(s_), ctypes.byref(c_))
    if kind < 1:
        raise SystemExit(f"{cfg.name} does not take the balanced path")
    waves = w_.value
    flag = {"auto": 0, "fused": cabi.QD_STAGE_FUSED, "unfused": cabi.QD_STAGE_UNFUSED}[args.merge]
    fused = args.merge == "fused" or (args.merge == "auto" and kind == 2)
    ws = cabi.auto_workspace(cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.block_size,
                             table.shape[1], dt, dev)
    out = torch.empty_like(q)
    buf = torch.zeros(waves * 16, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream(dev)
    scale = 1.0 / math.sqrt(cfg.head_dim)

    def launch(i, stamped):
        L.qd_diag_set_stamps(buf.data_ptr() if stamped else None)
        rc = L.qd_gqa_decode_auto_stages(q.data_ptr(), ks[i % pools].data_ptr(), vs[i % pools].data_ptr(),
                                         table.data_ptr(), lens.data_ptr(), out.data_ptr(), ws.data_ptr(),
                                         ws.numel(), cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim,
                                         cfg.block_size, table.shape[1], k.shape[0], dt, scale,
                                         cabi.QD_STAGE_ALL | flag, stream.cuda_stream)
        if rc:
            raise RuntimeError(L.qd_error_string(rc).decode())

    for i in range(args.warmup):
        launch(i, False)
    torch.cuda.synchronize()
    log(f"stamps: {cfg.name} waves={waves} fused={fused} launches={args.launches}")
    for n in range(args.launches):
        buf.zero_()
        torch.cuda.synchronize()
        launch(n, True)
        torch.cuda.synchronize()
        s = buf.view(waves, 16).cpu().tolist()
        t0 = min(r[0] for r in s)
        us = lambda x: (x - t0) / 100.0  # noqa: E731  (100 MHz ticks)
        ran = [r for r in s if r[1]]  # waves that held work
        ends = []
        for r in s:
            last = max(r[0], r[1], r[2], r[3], r[4], r[5])
            ends.append(us(last))
        rec = {"launch": n, "config": cfg.name, "fused": fused, "waves": waves, "waves_with_work": len(ran),
               "entry_max_us": round(max(us(r[0]) for r in s), 2),
               "prologue_end_us": {"p50": round(_pct([us(r[1]) for r in ran], .5), 2),
                                   "p90": round(_pct([us(r[1]) for r in ran], .9), 2)},
               "stream_end_us": {q_: round(_pct([us(r[2]) for r in ran], x), 2)
                                 for q_, x in (("p10", .1), ("p50", .5), ("p90", .9), ("max", 1.0))},
               "last_wave_end_us": round(max(ends), 2)}
        arr = [r for r in ran if r[3]]
        if arr:
            rec["store_retire_us"] = {"p50": round(_pct([(r[3] - r[2]) / 100 for r in arr], .5), 2),
                                      "max": round(max((r[3] - r[2]) / 100 for r in arr), 2)}
            rec["arrival_atomic_us"] = {"p50": round(_pct([(r[4] - r[3]) / 100 for r in arr], .5), 2),
                                        "max": round(max((r[4] - r[3]) / 100 for r in arr), 2)}
            mg = [r for r in arr if r[7] > 0]
            if mg:
                rec["merge_us"] = {"p50": round(_pct([(r[5] - r[4]) / 100 for r in mg], .5), 2),
                                   "max": round(max((r[5] - r[4]) / 100 for r in mg), 2), "merging_waves": len(mg)}
                rec["merge_start_us"] = {"p10": round(_pct([us(r[4]) for r in mg], .1), 2),
                                         "p50": round(_pct([us(r[4]) for r in mg], .5), 2),
                                         "max": round(max(us(r[4]) for r in mg), 2)}
        xcd = {}
        for r in ran:
            xcd.setdefault(int(r[6]), []).append(us(r[2]))
        rec["stream_end_p50_by_xcd_us"] = {str(x): round(_pct(v_, .5), 2) for x, v_ in sorted(xcd.items())}
        # Shader clock of each XCD over its waves' streaming: s_memtime ticks
        # per s_memrealtime tick (100 MHz), in MHz.
        clk = {}
        for r in ran:
            if r[2] > r[0] and r[9] > r[8]:
                clk.setdefault(int(r[6]), []).append((r[9] - r[8]) / ((r[2] - r[0]) / 100.0))
        rec["shader_mhz_by_xcd"] = {str(x): round(_pct(v_, .5), 1) for x, v_ in sorted(clk.items())}
        print(json.dumps(rec), flush=True)


def mla_stamps_mode(args) -> None:
    """Per-wave s_memrealtime stamps (100 MHz) of mla_attend_shared_kernel
    from attention_amd/lib/libqd_attention_diag.so (mla.hip built with
    -DQD_STAMPS) on --mla-config: entry, end of the prologue (partition and
    tile list), loop start (first tile and query landed), end of the last
    tile, and the XCD; tiles per range and the shader clocks spent in row
    ends.  The attention stage (qd_mla_attend: kernel + merge) is timed from
    the same library with the stamps off (median of 5 samples), then
    --launches launches are recorded one at a time over rotated caches; one
    JSON line per launch, microseconds from the first wave's entry."""
    import ctypes
    import attention_amd
    from attention_amd import _build, cabi
    from attention_amd.cases import MLA_CONFIGS

    L = ctypes.CDLL(_build.DIAG_LIB)
    V, I, I64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
    L.qd_diag_set_mla_stamps.argtypes = [V]
    L.qd_mla_attend.argtypes = [V] * 9 + [ctypes.c_size_t] + [I] * 7 + [I64, I, I, I, F, I, I, V]
    L.qd_mla_attend_workspace_bytes.restype = ctypes.c_size_t
    L.qd_mla_attend_workspace_bytes.argtypes = [I] * 11
    L.qd_mla_attend_info.argtypes = [I] * 11 + [ctypes.POINTER(I)] * 2
    L.qd_error_string.restype = ctypes.c_char_p
    cfg = MLA_CONFIGS[args.mla_config]
    dev = torch.device("cuda:0")
    c = {k: (v.to(dev) if v is not None else None) for k, v in cfg.make(device="cpu").items()}
    B, H = cfg.batch, cfg.heads
    Dn, Dc, Dr, P = cfg.nope_dim, cfg.latent_dim, cfg.rope_dim, cfg.block_size
    dt = cabi.DTYPE[cfg.dtype]
    table, lens, pos = c["table"], c["lens"], c["positions"]
    s_, g_ = I(), I()
    kind = L.qd_mla_attend_info(B, 1, H, Dc, Dr, P, table.shape[1], -1, dt, 0, 0, ctypes.byref(s_), ctypes.byref(g_))
    if kind != 3:
        raise SystemExit(f"{cfg.name} does not take the shared-tile kernel (kind {kind})")
    esz = c["cache"].element_size()
    pools = args.pools or max(2, math.ceil(768e6 / (c["cache"].numel() * esz)))
    caches = [c["cache"]] + [c["cache"].roll(i, dims=0).contiguous() for i in range(1, pools)]
    scale = 1.0 / math.sqrt(Dn + Dr)
    qa = attention_amd.mla_query_absorb(c["q_nope"], c["w_uk"])
    out = torch.empty(B, 1, H, Dc, dtype=cfg.dtype, device=dev)
    need = L.qd_mla_attend_workspace_bytes(B, 1, H, Dc, Dr, P, table.shape[1], -1, dt, 0, 0)
    ws = torch.empty(max(16, need), dtype=torch.uint8, device=dev)
    grid = ((s_.value + 7) // 8) * 8 * g_.value
    buf = torch.zeros(grid * 4 * 16, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream(dev)

    def attend(i):
        rc = L.qd_mla_attend(qa.data_ptr(), c["q_rope"].data_ptr(), caches[i % pools].data_ptr(), table.data_ptr(),
                             lens.data_ptr(), pos.data_ptr(), None, out.data_ptr(), ws.data_ptr(), ws.numel(),
                             B, 1, H, Dc, Dr, P, table.shape[1], caches[0].shape[0], -1, 1, dt, scale, 0, 0,
                             stream.cuda_stream)
        if rc:
            raise RuntimeError(L.qd_error_string(rc).decode())

    L.qd_diag_set_mla_stamps(None)
    samples = time_samples(attend, args.steps, args.warmup, stream)
    log(f"mla stamps: {cfg.name} workgroups={s_.value} head_groups={g_.value} pools={pools}; attention stage "
        f"(stamps off) {statistics.median(samples) * 1e3:.2f} us median of {len(samples)} samples")
    for n in range(args.launches):
        buf.zero_()
        L.qd_diag_set_mla_stamps(buf.data_ptr())
        torch.cuda.synchronize()
        attend(n)
        torch.cuda.synchronize()
        L.qd_diag_set_mla_stamps(None)
        rows = [r for r in buf.view(-1, 16).cpu().tolist() if r[0]]
        t0 = min(r[0] for r in rows)
        us = lambda x: (x - t0) / 100.0  # noqa: E731  (100 MHz ticks)
        mhz = statistics.median([(r[9] - r[8]) / ((r[3] - r[0]) / 100.0) for r in rows if r[3] > r[0]])
        loop_tile = [((r[3] - r[2]) / 100.0 - r[7] / mhz) / max(1, r[6]) for r in rows]
        xcd = {}
        for r in rows:
            xcd.setdefault(int(r[5]), []).append(us(r[3]))

        def pct(key, qs):
            vals = [key(r) for r in rows]
            return {q_: round(_pct(vals, x), 2) for q_, x in qs}
        rec = {"launch": n, "config": cfg.name, "waves": len(rows), "shader_mhz": round(mhz, 1),
               "prologue_end_us": pct(lambda r: us(r[1]), (("p50", .5), ("p90", .9))),
               "loop_start_us": pct(lambda r: us(r[2]), (("p50", .5), ("p90", .9))),
               "loop_end_us": pct(lambda r: us(r[3]), (("p10", .1), ("p50", .5), ("p90", .9), ("max", 1.0))),
               "kernel_end_max_us": round(max(us(r[4]) for r in rows), 2),
               "tiles_per_range": {"min": min(r[6] for r in rows), "p50": round(_pct([r[6] for r in rows], .5)),
                                   "max": max(r[6] for r in rows)},
               "row_end_us_per_wave": pct(lambda r: r[7] / mhz, (("p50", .5), ("max", 1.0))),
               "loop_us_per_tile_excluding_row_ends": {"p50": round(_pct(loop_tile, .5), 3),
                                                       "cycles": round(_pct(loop_tile, .5) * mhz)},
               "loop_end_p50_by_xcd_us": {str(x): round(_pct(v_, .5), 2) for x, v_ in sorted(xcd.items())}}
        print(json.dumps(rec), flush=True)


def read_mode(args) -> None:
    """The HBM read ceiling for the decode kernel's bytes: the probes of
    attention_amd/lib/libqd_attention_diag.so (stream_probe.hip) over the
    config's own K/V pools (head_dim 128, 16-bit), rotated as in the decode
    bench.  `paged`: the decode kernel's loads without its math, partition
    or merge (one workgroup of kv_heads waves per CU, whole 16-token groups
    of the shuffled pages, two groups in flight, nontemporal 16-byte loads);
    `linear`: a contiguous read of the same pools.  Median of 5 samples; the
    decode floor is the decode call's algorithmic bytes at the paged rate."""
    import ctypes
    from attention_amd import _build
    from attention_amd.cases import algorithmic_bytes, get_config

    L = ctypes.CDLL(_build.DIAG_LIB)
    V, I, I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    L.qd_diag_stream_read.argtypes = [V, V, V, I64, I, I, I, I, I, I, I, I, V, V, V]
    cfg = get_config(args.config)
    if cfg.head_dim != 128 or cfg.dtype not in (torch.float16, torch.bfloat16):
        raise SystemExit("--mode read covers 16-bit caches with head_dim 128")
    dev = torch.device("cuda:0")
    lengths = cfg.lengths()
    case = (cfg.make(device=dev, device_gen=True, lengths=lengths) if args.device_gen
            else tuple(x.to(dev) for x in cfg.make(device="cpu", lengths=lengths)))
    q, k, v, table, lens = case
    kv_bytes = 2 * k.numel() * k.element_size()
    pools = args.pools or max(2, math.ceil(768e6 / kv_bytes))
    ks, vs = [k], [v]
    for i in range(1, pools):
        ks.append(k.roll(i, dims=0).contiguous())
        vs.append(v.roll(i, dims=0).contiguous())
    # Every page of the exact pool, in the page table's order (sequence by
    # sequence): the shuffled physical order the decode kernel visits.
    used = [table[b, :math.ceil(n / cfg.block_size)] for b, n in enumerate(lengths) if n > 0]
    pages = torch.cat(used).to(torch.int32).contiguous()
    npages = pages.numel()
    assert int(pages.min()) >= 0 and int(pages.max()) < k.shape[0]
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    waves = min(cfg.kv_heads, 8) * args.probe_split
    if waves > 8:
        raise SystemExit("--probe-split 2 needs at most 4 kv-heads")
    wgs = cus
    sink = torch.empty(wgs * waves * 64, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    probe_bytes = 2 * npages * cfg.block_size * cfg.kv_heads * cfg.head_dim * k.element_size()
    res = {}
    for name, mode in (("paged", 0), ("linear", 1)):
        def step(i, mode=mode):
            rc = L.qd_diag_stream_read(ks[i % pools].data_ptr(), vs[i % pools].data_ptr(), pages.data_ptr(),
                                       npages, cfg.block_size, cfg.kv_heads, wgs, waves, mode, args.probe_pf,
                                       args.probe_work, args.probe_split, sink.data_ptr(), None,
                                       stream.cuda_stream)
            if rc:
                raise RuntimeError(f"qd_diag_stream_read failed: {rc}")
        samples = time_samples(step, args.steps, args.warmup, stream)
        ms = statistics.median(samples)
        res[name] = {"us_per_launch": round(ms * 1e3, 3), "tbs": round(probe_bytes / (ms * 1e-3) / 1e12, 4),
                     "samples_us": [round(x * 1e3, 3) for x in samples]}
        log(f"{name}: {ms * 1e3:.2f} us, {probe_bytes / (ms * 1e-3) / 1e12:.3f} TB/s")
    # Per-wave end stamps of single paged launches, one per pool: the spread
    # of the workgroups' end times by XCD with no decode work at all.
    stamps = torch.zeros(wgs * waves * 4, dtype=torch.int64, device=dev)
    by_pool = []
    for i in range(pools):
        stamps.zero_()
        torch.cuda.synchronize()
        rc = L.qd_diag_stream_read(ks[i].data_ptr(), vs[i].data_ptr(), pages.data_ptr(), npages, cfg.block_size,
                                   cfg.kv_heads, wgs, waves, 0, args.probe_pf, args.probe_work, args.probe_split,
                                   sink.data_ptr(), stamps.data_ptr(), stream.cuda_stream)
        if rc:
            raise RuntimeError(f"qd_diag_stream_read failed: {rc}")
        torch.cuda.synchronize()
        s = stamps.view(-1, 4).cpu().tolist()
        t0 = min(r[0] for r in s)
        ends = [(r[1] - t0) / 100.0 for r in s]
        xcd = {}
        for r, e in zip(s, ends):
            xcd.setdefault(int(r[2]), []).append(e)
        by_pool.append({"pool": i, "end_us": {"p10": round(_pct(ends, .1), 2), "p50": round(_pct(ends, .5), 2),
                                              "max": round(max(ends), 2)},
                        "end_p50_by_xcd_us": {str(x): round(_pct(v_, .5), 2) for x, v_ in sorted(xcd.items())}})
        log(f"paged probe, pool {i}: end p50 {by_pool[-1]['end_us']['p50']} max {by_pool[-1]['end_us']['max']} us; "
            f"by XCD {by_pool[-1]['end_p50_by_xcd_us']}")
    res["paged"]["stamps_by_pool"] = by_pool
    alg = algorithmic_bytes(lengths, cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.block_size,
                            q.element_size())
    rate = res["paged"]["tbs"] * 1e12
    print(json.dumps({"mode": "read", "config": cfg.name, "bytes_read_per_launch": probe_bytes,
                      "probe_groups_in_flight": args.probe_pf, "probe_work_per_group": args.probe_work,
                      "probe_split": args.probe_split,
                      "pages": npages, "workgroups": wgs, "waves_per_workgroup": waves, "pools_rotated": pools,
                      "paged": res["paged"], "linear": res["linear"], "peak_tbs": PEAK_HBM_GBS / 1e3,
                      "decode_algorithmic_bytes": alg,
                      "decode_floor_us_at_paged_rate": round(alg / rate * 1e6, 2),
                      "target_us_at_80pct_of_peak": round(alg / (0.8 * PEAK_HBM_GBS * 1e9) * 1e6, 2)}), flush=True)


def cpu_threads() -> tuple[int, dict]:
    """Threads for the CPU baseline and what they were derived from.

    The baseline's plan is one thread per host core (``os.cpu_count()``).  A
    job on the GPU box is confined to its CPU share (its affinity mask) and
    gets ``OMP_NUM_THREADS`` set to that share, so the thread count is the
    smallest of the three: more threads than the cores the process may run
    on would time oversubscription, not the reference path."""
    counts = {"os_cpu_count": os.cpu_count() or 1}
    try:
        counts["affinity_cpus"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        counts["affinity_cpus"] = counts["os_cpu_count"]
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        counts["omp_num_threads"] = int(omp)
    return min(counts.values()), counts


def _time_cpu(fn, repeats: int, min_s: float, max_s: float) -> list[float]:
    """1 warmup call, then timed calls until there are at least `repeats`
    of them over at least `min_s` seconds, or `max_s` seconds have passed."""
    fn()
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        spent = time.perf_counter() - t_start
        if (len(times) >= repeats and spent >= min_s) or spent >= max_s:
            break
    return times


def _rss_gb() -> float:
    import resource
    return resource.getrusage(resource.RUSAGE_SELF).ru_maxrss / 1e6  # ru_maxrss is in KiB on Linux


def other_cpu_configs(skip: str) -> dict:
    """One timed call of the reference CPU path on each other BASELINE config
    (the baseline plan's cfg2-cfg5 once each): cfg3 and cfg5 on their whole
    batches; cfg4 on its first sequence only, because the path materializes
    about len*Hq*D*4 bytes each for repeated K and V in fp32 (up to 4.3 GB
    each per sequence) and the whole batch would take about a minute of the
    bench.  Peak host memory (max RSS) is logged after each."""
    from oracle.cpu_path import reference_cpu_path
    from attention_amd.cases import CONFIGS, algorithmic_bytes, make_decode_case

    out = {}
    for name in ("cfg3", "cfg5", "cfg4"):
        if name == skip:
            continue
        c = CONFIGS[name]
        lengths = c.lengths()
        note = "whole batch"
        if name == "cfg4":
            lengths = lengths[:1]
            note = (f"first sequence only ({lengths[0]} tokens of the batch's {sum(c.lengths())}): the whole "
                    "batch would materialize up to 8.6 GB of fp32 K/V per sequence for about a minute")
            case = make_decode_case(lengths=lengths, q_heads=c.q_heads, kv_heads=c.kv_heads, head_dim=c.head_dim,
                                    block_size=c.block_size, dtype=c.dtype, seed=c.seed, exact_pool=True,
                                    k_scale=c.k_scale)
        else:
            case = c.make(device="cpu", lengths=lengths)
        t0 = time.perf_counter()
        reference_cpu_path(*case)
        t = time.perf_counter() - t0
        nbytes = algorithmic_bytes(lengths, len(lengths), c.q_heads, c.kv_heads, c.head_dim, c.block_size,
                                   case[0].element_size())
        out[name] = {"us_per_call": round(t * 1e6, 1), "gb_s": round(nbytes / t / 1e9, 3), "sequences": len(lengths),
                     "tokens": sum(lengths), "sample": note, "max_rss_gb": round(_rss_gb(), 2)}
        log(f"cpu baseline {name}: {t * 1e3:.1f} ms ({note}), {nbytes / t / 1e9:.3f} GB/s, "
            f"max RSS {_rss_gb():.1f} GB")
        del case
    return out


def cpu_baseline(case_cpu, cfg, repeats: int, other_configs: bool = True) -> dict:
    """Times the reference CPU path (oracle/cpu_path.py, the torch CPU ops of
    reference attention/reference/gqa.py:21-44) on the host cores: the whole
    batch of the benchmark config, and cfg1 (the reference's own
    CPU-runnable config, which the baseline plan requires)."""
    from oracle.cpu_path import reference_cpu_path
    from attention_amd.cases import CONFIGS, algorithmic_bytes

    threads, counts = cpu_threads()
    torch.set_num_threads(threads)
    q, k, v, table, lens = case_cpu
    lens_l = lens.tolist()
    times = _time_cpu(lambda: reference_cpu_path(q, k, v, table, lens), max(5, repeats), 10.0, 30.0)
    t = statistics.median(times)
    b_full = algorithmic_bytes(lens_l, len(lens_l), cfg.q_heads, cfg.kv_heads, cfg.head_dim,
                               cfg.block_size, q.element_size())
    c1 = CONFIGS["cfg1"]
    case1 = c1.make(device="cpu")
    t1 = statistics.median(_time_cpu(lambda: reference_cpu_path(*case1), 50, 2.0, 10.0))
    others = other_cpu_configs(skip=cfg.name) if other_configs else {}
    return {"value": round(b_full / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_call": round(t * 1e6, 1),
            "cfg1_us_per_call": round(t1 * 1e6, 1),
            "other_configs": others,
            "sample": (f"oracle/cpu_path.reference_cpu_path (torch CPU ops of reference "
                       f"attention/reference/gqa.py:21-44) on the whole {cfg.name} batch "
                       f"({len(lens_l)} sequences, {sum(lens_l)} tokens, the same input as the GPU "
                       f"run), median of {len(times)} calls after 1 warmup ({sum(times):.1f} s): "
                       f"{t * 1e3:.1f} ms per call; cfg1 (lens 17/100/255/512): "
                       f"{t1 * 1e6:.0f} us per call"),
            "threads_from": counts,
            "cpu": _cpu_model()}


def profiled_traffic(kernel: str, config: str):
    """HBM bytes per dispatch of `kernel` on `config` from the committed
    rocprofv3 counter summary (profiles/<kernel>_<config>_traffic.txt, line
    'traffic_bytes_per_dispatch: N'), or None when there is none."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_{config}_traffic.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_dispatch:"):
                    return int(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def kv_append_mode(args) -> None:
    """One step = one attention_amd.kv_append call writing one token per
    sequence of the config (positions = length - 1, rotating over cache
    pools above the Infinity Cache size).  Bytes = key+value read and the
    two cache rows written per sequence, plus the table entry and position."""
    import attention_amd
    from attention_amd.cases import get_config

    cfg = get_config(args.config)
    dev = torch.device("cuda:0")
    lengths = cfg.lengths()
    _, k, v, table, lens = cfg.make(device=dev, device_gen=True, lengths=lengths)
    B, Hkv, D = cfg.batch, cfg.kv_heads, cfg.head_dim
    gen = torch.Generator(device=dev).manual_seed(7)
    key = torch.randn(B, Hkv, D, device=dev, generator=gen).to(cfg.dtype)
    value = torch.randn(B, Hkv, D, device=dev, generator=gen).to(cfg.dtype)
    pos = (lens - 1).clamp(min=0).to(torch.int32)
    kv_bytes = 2 * k.numel() * k.element_size()
    pools = max(2, math.ceil(768e6 / kv_bytes))
    ks, vs = [k], [v]
    for _ in range(1, pools):
        ks.append(torch.empty_like(k))
        vs.append(torch.empty_like(v))
    stream = torch.cuda.current_stream(dev)
    ms = time_loop(lambda i: attention_amd.kv_append(key, value, ks[i % pools], vs[i % pools], table, pos),
                   args.steps, args.warmup, stream)
    s = key.element_size()
    nbytes = 4 * B * Hkv * D * s + 8 * B
    gbs = nbytes / (ms * 1e-3) / 1e9
    # CPU baseline: the reference's comparator, torch indexed assignment
    # (benchmarks/bench_all_operators.py:100-102), on the host copies.
    kc, vc, tc, pc, kk, vv = (x.cpu() for x in (k, v, table, pos, key, value))
    idx = torch.arange(B)
    page, slot = tc[idx, (pc // cfg.block_size).long()].long(), (pc % cfg.block_size).long()
    times = []
    for _ in range(max(5, args.cpu_repeats)):
        t0 = time.perf_counter()
        kc[page, slot] = kk
        vc[page, slot] = vv
        times.append(time.perf_counter() - t0)
    t_cpu = statistics.median(times)
    print(json.dumps({
        "metric": "paged KV append µs/call and achieved HBM GB/s, 1 MI355X",
        "value": round(gbs, 2), "unit": "GB/s", "us_per_call": round(ms * 1e3, 3),
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 6),
        "higher_is_better": True, "dtype": DT_NAME[cfg.dtype], "data": "synthetic",
        "config": {"workload": f"kv_append on {cfg.name} shapes", "batch": B, "kv_heads": Hkv,
                   "head_dim": D, "block_size": cfg.block_size, "bytes_per_call": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 5), "traffic": None,
                     "note": "launch-bound: one token per sequence is a few hundred KB"},
        "cpu_baseline": {"value": round(nbytes / t_cpu / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
                         "kind": "port", "sample": f"torch indexed assignment on CPU, median {t_cpu * 1e6:.1f} us"},
    }), flush=True)


def sweep_mode(args) -> None:
    """The reference's own decode measurement (benchmarks/measure_decode.py:
    43-57): attention.gqa_decode on make_decode_case(lengths=[L]*B,
    Hq32/Hkv8/D128/P16, seed 42, pool B*max_pages blocks) for fp32, fp16 and
    bf16, B in {1, 4, 16}, L in {128, 1024, 4096}; 20 warmup calls, then 5
    samples of 10 calls (HIP events, output allocation included), median
    us per call.  The inputs are not rotated, as in the reference, so the
    smaller points are served partly from the Infinity Cache.  Each point also
    reports `gpu_us`: the same call through the C entry point on a
    preallocated workspace, 10 calls captured in a HIP graph and replayed
    (graph_replay_us), which leaves out the host's per-call cost.  One JSON
    line per point, then a summary line."""
    import attention_amd
    from attention_amd import cabi
    from attention_amd.cases import algorithmic_bytes, make_decode_case

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    rows = []
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        for batch in (1, 4, 16):
            for length in (128, 1024, 4096):
                inputs = make_decode_case(lengths=[length] * batch, q_heads=32, kv_heads=8, head_dim=128,
                                          block_size=16, dtype=dtype, device=dev)
                maxp = inputs[3].shape[1]
                kind, waves, _, _ = cabi.auto_info(batch, 32, 8, 128, 16, maxp, cabi.DTYPE[dtype])
                samples = time_samples(lambda i: attention_amd.gqa_decode(*inputs), 10, 20, stream)
                med = statistics.median(samples)
                ws = cabi.auto_workspace(batch, 32, 8, 128, 16, maxp, cabi.DTYPE[dtype], dev)
                out = torch.empty_like(inputs[0])

                def enqueue():
                    rc = cabi.auto_launch(*inputs, out, scale=1 / math.sqrt(128), workspace=ws,
                                          stream=torch.cuda.current_stream(dev).cuda_stream)
                    if rc != 0:
                        raise RuntimeError(cabi.error_string(rc))

                gpu_us = graph_replay_us(enqueue, stream)
                nbytes = algorithmic_bytes([length] * batch, batch, 32, 8, 128, 16, inputs[0].element_size())
                row = {"dtype": DT_NAME[dtype], "batch": batch, "length": length, "hq": 32, "hkv": 8,
                       "head_dim": 128, "block_size": 16, "median_us": round(med * 1e3, 3),
                       "min_us": round(min(samples) * 1e3, 3), "max_us": round(max(samples) * 1e3, 3),
                       "gpu_us": round(gpu_us, 3), "waves": waves,
                       "gb_s": round(nbytes / (med * 1e-3) / 1e9, 1),
                       "path": {1: "balanced MFMA + merge", 2: "balanced MFMA, fused merge",
                                0: "split layout"}.get(kind, "?")}
                rows.append(row)
                print(json.dumps(row), flush=True)
                del inputs, ws, out
    print(json.dumps({"op": "sweep", "points": len(rows),
                      "method": "20 warmup, 5 samples x 10 calls, median (measure_decode.py:47-57)",
                      "median_us": {f"{r['dtype']}/B{r['batch']}/L{r['length']}": r["median_us"] for r in rows},
                      "gpu_us": {f"{r['dtype']}/B{r['batch']}/L{r['length']}": r["gpu_us"] for r in rows}}),
          flush=True)


# Decode shapes of common model families (q_heads, kv_heads, head_dim), bf16,
# 16-token pages: the Hq/Hkv/D of each model's attention (the tensor-parallel
# share where named), and the batch x context points they are timed at.
MODEL_SHAPES = {
    "llama3.2-1b": (32, 8, 64),
    "qwen2.5-0.5b": (14, 2, 64),
    "tinyllama-1.1b": (32, 4, 64),
    "qwen2.5-7b": (28, 4, 128),
    "mistral-7b": (32, 8, 128),
    "llama2-7b": (32, 32, 128),
    "llama3-70b-tp8": (8, 1, 128),
    "gemma2-9b": (16, 8, 256),
    "gemma2-2b": (8, 4, 256),
    "phi3-mini": (32, 32, 96),
    "qwen3-30b-a3b": (32, 4, 128),
}
MODEL_POINTS = ((32, 4096), (128, 1024), (8, 8192))


def models_mode(args) -> None:
    """The automatic path on the shapes of MODEL_SHAPES at MODEL_POINTS
    (make_decode_case, bf16, P16, equal lengths): GPU time per call from graph
    replays of the C entry point (graph_replay_us; 10 calls captured over K/V
    pools rotated above 768 MB, so the Infinity Cache does not serve them),
    algorithmic GB/s and the share of 8 TB/s.  Without --model, each shape
    runs in a child process of its own (this process never touches the GPU):
    in one process, a shape allocated after a larger one was freed measured
    up to 25% slower.  One JSON line per point."""
    if not args.model:
        import subprocess
        for name in MODEL_SHAPES:
            res = subprocess.run([sys.executable, os.path.abspath(__file__), "--op", "models", "--model", name],
                                 stdout=subprocess.PIPE, text=True, timeout=300)
            sys.stdout.write(res.stdout)
            sys.stdout.flush()
            if res.returncode != 0:
                raise SystemExit(f"--op models --model {name} failed ({res.returncode})")
        return
    from attention_amd import cabi
    from attention_amd.cases import algorithmic_bytes, make_decode_case

    if args.model not in MODEL_SHAPES:
        raise SystemExit(f"--model: one of {', '.join(MODEL_SHAPES)}")
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    hq, hkv, d = MODEL_SHAPES[args.model]
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    dt = torch.bfloat16
    for batch, length in MODEL_POINTS:
        q, k, v, table, lens = make_decode_case(lengths=[length] * batch, q_heads=hq, kv_heads=hkv, head_dim=d,
                                                block_size=16, dtype=dt, device=dev)
        kv_bytes = 2 * k.numel() * k.element_size()
        pools = max(1, math.ceil(768e6 / kv_bytes))
        ks, vs = [k], [v]
        for i in range(1, pools):
            ks.append(k.roll(i, dims=0).contiguous())
            vs.append(v.roll(i, dims=0).contiguous())
        maxp = table.shape[1]
        kind, waves, _, _ = cabi.auto_info(batch, hq, hkv, d, 16, maxp, cabi.DTYPE[dt])
        ws = cabi.auto_workspace(batch, hq, hkv, d, 16, maxp, cabi.DTYPE[dt], dev)
        out = torch.empty_like(q)
        turn = [0]

        def enqueue():
            i = turn[0] % pools
            turn[0] += 1
            rc = cabi.auto_launch(q, ks[i], vs[i], table, lens, out, scale=1 / math.sqrt(d), workspace=ws,
                                  stream=torch.cuda.current_stream(dev).cuda_stream)
            if rc:
                raise RuntimeError(cabi.error_string(rc))

        us = graph_replay_us(enqueue, stream)
        nb = algorithmic_bytes([length] * batch, batch, hq, hkv, d, 16, 2)
        print(json.dumps({"model": args.model, "q_heads": hq, "kv_heads": hkv, "head_dim": d, "batch": batch,
                          "len": length, "path": "balanced MFMA + merge" if kind >= 1 else "split layout",
                          "waves": waves if kind >= 1 else None, "pools": pools, "gpu_us": round(us, 2),
                          "gbs": round(nb / us / 1e3, 1), "pct_of_8tbs": round(nb / us / 8e4, 1),
                          "mb": round(nb / 1e6, 1)}), flush=True)
        del q, k, v, table, lens, ks, vs, ws, out
        torch.cuda.empty_cache()


def splits_mode(args) -> None:
    """The split layout (decode_generic_kernel + the split merge) by split
    count, on fp32 shapes of the reference's sweep (Hq32/Hkv8/D128/P16,
    make_decode_case seed 42) and a longer one: GPU time per call from graph
    replays of the C entry point (graph_replay_us) for split counts 8..512
    (whole pages per split), with the plan's choice (qd_gqa_decode_plan)
    marked.  One JSON line per shape."""
    from attention_amd import cabi
    from attention_amd.cases import make_decode_case

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    f32 = cabi.DTYPE[torch.float32]
    for batch, length in ((1, 1024), (1, 4096), (4, 1024), (4, 4096), (16, 1024), (16, 4096), (1, 16384)):
        inputs = make_decode_case(lengths=[length] * batch, q_heads=32, kv_heads=8, head_dim=128, block_size=16,
                                  dtype=torch.float32, device=dev)
        maxp = inputs[3].shape[1]
        plan_s, plan_c = cabi.plan(batch, 32, 8, 128, 16, maxp, f32)
        out = torch.empty_like(inputs[0])
        times = {}
        for want in sorted({plan_s, 8, 16, 32, 64, 128, 256, 512}):
            if want > maxp:
                continue
            chunk = plan_c if want == plan_s else -(-maxp // want)
            splits = -(-maxp // chunk)
            ws = torch.empty(batch * 32 * splits * 130, dtype=torch.float32, device=dev)

            def enqueue():
                rc = cabi.launch(*inputs, out, scale=1 / math.sqrt(128), splits=splits, chunk_pages=chunk,
                                 workspace=ws, stream=torch.cuda.current_stream(dev).cuda_stream)
                if rc != 0:
                    raise RuntimeError(cabi.error_string(rc))

            times[f"S{splits}x{chunk}p"] = round(graph_replay_us(enqueue, stream), 3)
            del ws
        best = min(times, key=times.get)
        print(json.dumps({"dtype": "fp32", "batch": batch, "length": length, "plan": f"S{plan_s}x{plan_c}p",
                          "gpu_us": times, "fastest": best}), flush=True)
        del inputs, out


PEAK_MFMA_BF16_TFLOPS = 2500.0


def mla_mode(args) -> None:
    """One step = one attention_amd.mla_decode call (query absorption, paged
    latent attention, value projection) over the batch of --mla-config, with
    caches and weights rotated over pools above the Infinity Cache size.
    value = algorithmic HBM bytes of the call / time: visible cache rows
    once, q_nope and q_rope, both weight tensors, the output, lengths,
    positions and used table entries.  The roofline is the latent-attention
    stage alone (qd_mla_attend: attention kernel, plus the split merge when
    the plan splits), on the absorbed query."""
    import attention_amd
    from attention_amd import cabi
    from attention_amd.cases import MLA_CONFIGS, mla_attend_bytes

    cfg = MLA_CONFIGS[args.mla_config]
    dev = torch.device("cuda:0")
    t0 = time.perf_counter()
    lengths = cfg.lengths()
    c_cpu = cfg.make(device="cpu")
    c = {k: (v.to(dev) if v is not None else None) for k, v in c_cpu.items()}
    B, H = cfg.batch, cfg.heads
    Dn, Dc, Dr, Dv, P = cfg.nope_dim, cfg.latent_dim, cfg.rope_dim, cfg.value_dim, cfg.block_size
    s = c["cache"].element_size()
    per_pool = (c["cache"].numel() + c["w_uk"].numel() + c["w_uv"].numel()) * s
    pools = args.pools or max(2, math.ceil(768e6 / per_pool))
    caches, wks, wvs = [c["cache"]], [c["w_uk"]], [c["w_uv"]]
    for i in range(1, pools):
        caches.append(c["cache"].roll(i, dims=0).contiguous())
        wks.append(c["w_uk"].roll(i, dims=0).contiguous())
        wvs.append(c["w_uv"].roll(i, dims=0).contiguous())
    table, lens, pos = c["table"], c["lens"], c["positions"]
    scale = 1.0 / math.sqrt(Dn + Dr)
    torch.cuda.synchronize()
    log(f"{cfg.name}: {B} seqs, sum len {sum(lengths)}, cache {c['cache'].numel() * s / 1e6:.1f} MB, "
        f"weights {(c['w_uk'].numel() + c['w_uv'].numel()) * s / 1e6:.1f} MB x {pools} pools, "
        f"setup {time.perf_counter() - t0:.1f}s")
    stream = torch.cuda.current_stream(dev)

    if args.splits:
        out = torch.empty(B, 1, H, Dv, dtype=cfg.dtype, device=dev)

        def step(i):
            rc = cabi.mla_decode(c["q_nope"], c["q_rope"], caches[i % pools], table, lens, pos, wks[i % pools],
                                 wvs[i % pools], out, scale=scale, splits=args.splits)
            if rc:
                raise RuntimeError(cabi.error_string(rc))
        path = f"C ABI qd_mla_decode splits={args.splits}"
    else:
        def step(i):
            attention_amd.mla_decode(c["q_nope"], c["q_rope"], caches[i % pools], table, lens, pos,
                                     wks[i % pools], wvs[i % pools])
        path = "attention_amd.mla_decode (torch.ops.qd_attention.mla_decode_fused)"
    ms = time_loop(step, args.steps, args.warmup, stream)
    rows = sum(lengths)
    meta = 4 * B + 4 * B + 4 * sum(math.ceil(x / P) for x in lengths)
    call_bytes = (rows * (Dc + Dr) * s + B * H * (Dn + Dr) * s + H * Dn * Dc * s + H * Dv * Dc * s
                  + B * H * Dv * s + meta)
    gbs = call_bytes / (ms * 1e-3) / 1e9
    log(f"mla_decode: {ms * 1e3:.2f} us/call, {gbs:.1f} GB/s algorithmic")

    # Latent attention alone, on the absorbed query.
    mflags = {"auto": 0, "wave": cabi.QD_FLAG_MLA_WAVE, "staged": cabi.QD_FLAG_MLA_STAGED}[args.mla_kernel]
    kind, splits, groups = cabi.mla_attend_info(B, 1, H, Dc, Dr, P, table.shape[1], -1, cabi.DTYPE[cfg.dtype],
                                                args.splits, mflags)
    qa = attention_amd.mla_query_absorb(c["q_nope"], c["w_uk"])
    lat = torch.empty(B, 1, H, Dc, dtype=cfg.dtype, device=dev)
    need = cabi.lib().qd_mla_attend_workspace_bytes(B, 1, H, Dc, Dr, P, table.shape[1], -1,
                                                    cabi.DTYPE[cfg.dtype], args.splits, mflags)
    ws = torch.empty(max(16, need), dtype=torch.uint8, device=dev)

    def attend(i):
        rc = cabi.mla_attend(qa, c["q_rope"], caches[i % pools], table, lens,
                             pos, lat, scale=scale, splits=args.splits, workspace=ws, flags=mflags,
                             stream=stream.cuda_stream)
        if rc:
            raise RuntimeError(cabi.error_string(rc))
    a_ms = time_loop(attend, args.steps, args.warmup, stream)
    a_bytes = mla_attend_bytes(lengths, 1, H, Dc, Dr, P, s)
    a_gbs = a_bytes / (a_ms * 1e-3) / 1e9
    a_flops = 2 * rows * H * (Dc + Dr + Dc)
    a_tflops = a_flops / (a_ms * 1e-3) / 1e12
    kname = {3: "mla_attend_shared_kernel", 2: "mla_attend_wave_kernel",
             1: "mla_attend_mfma_kernel"}.get(kind, "mla_attend_generic_kernel")
    if kind >= 1:
        kernels = kname + "+mla_merge_sk_kernel"
    else:
        kernels = kname + ("+mla_merge_kernel" if splits > 1 else "")
    log(f"{kernels}: {a_ms * 1e3:.2f} us, {a_gbs:.1f} GB/s ({100 * a_gbs / PEAK_HBM_GBS:.1f}% of HBM peak), "
        f"{a_tflops:.1f} TFLOP/s ({100 * a_tflops / PEAK_MFMA_BF16_TFLOPS:.1f}% of bf16 MFMA peak); "
        f"{'workgroups' if kind >= 1 else 'splits'}={splits} head_groups={groups}")
    result = {
        "metric": "paged MLA decode µs/call and achieved HBM GB/s, 1 MI355X",
        "value": round(gbs, 2), "unit": "GB/s", "us_per_call": round(ms * 1e3, 3),
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": DT_NAME[cfg.dtype],
        "data": "synthetic: seeded N(0,1) latent cache and queries, scaled N(0,1) weights, shuffled exact pool",
        "config": {"workload": f"{cfg.name}: {cfg.description}", "batch": B, "heads": H, "nope_dim": Dn,
                   "latent_dim": Dc, "rope_dim": Dr, "value_dim": Dv, "block_size": P,
                   "context_lens": f"U{list(cfg.len_range)}: sum {rows}, min {min(lengths)}, max {max(lengths)}",
                   "pools_rotated": pools, "path": path, "algorithmic_bytes_per_call": call_bytes},
        "roofline": {"bound": "hbm", "kernel": kernels, "achieved": round(a_gbs, 2), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(a_gbs / PEAK_HBM_GBS, 4),
                     "traffic": profiled_traffic(kname, cfg.name), "duration_us": round(a_ms * 1e3, 3),
                     "algorithmic_bytes": a_bytes, "mfma_tflops": round(a_tflops, 2),
                     "mfma_frac": round(a_tflops / PEAK_MFMA_BF16_TFLOPS, 4),
                     ("workgroups" if kind >= 1 else "splits"): splits, "head_groups": groups,
                     "note": "latent attention on the absorbed query (qd_mla_attend: attention kernel + merge of "
                             "rows split across workgroups), HIP events on its stream; "
                             f"{a_flops / a_bytes:.0f} flop/byte against a bf16 ridge of "
                             f"{PEAK_MFMA_BF16_TFLOPS / PEAK_HBM_GBS * 1e3:.0f}"},
    }
    if not args.no_cpu_baseline:
        from oracle.cpu_path import reference_mla_cpu_path
        threads, counts = cpu_threads()
        torch.set_num_threads(threads)
        nb = 2
        sample = [c_cpu[k][:nb] for k in ("q_nope", "q_rope")] + [c_cpu["cache"], c_cpu["table"][:nb],
                                                                  c_cpu["lens"][:nb], c_cpu["positions"][:nb],
                                                                  c_cpu["w_uk"], c_cpu["w_uv"]]
        reference_mla_cpu_path(*sample, scale=scale)
        times, t_start = [], time.perf_counter()
        while True:
            t1 = time.perf_counter()
            reference_mla_cpu_path(*sample, scale=scale)
            times.append(time.perf_counter() - t1)
            if (len(times) >= 3 and time.perf_counter() - t_start >= 10.0) or time.perf_counter() - t_start >= 30.0:
                break
        t = statistics.median(times)
        sb = (sum(lengths[:nb]) * (Dc + Dr) * s + nb * H * (Dn + Dr + Dv) * s + H * Dn * Dc * s
              + H * Dv * Dc * s)
        result["cpu_baseline"] = {
            "value": round(sb / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": (f"oracle/cpu_path.reference_mla_cpu_path (torch CPU ops of reference "
                       f"attention/reference/mla.py:6-34, absorbed) on the first {nb} of {B} sequences "
                       f"({sum(lengths[:nb])} tokens), median of {len(times)} calls: {t * 1e3:.1f} ms"),
            "threads_from": counts, "cpu": _cpu_model()}
    print(json.dumps(result), flush=True)


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> None:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the decode path is "
              "measured on one MI355X and multi-GPU sharding is design-only.", file=sys.stderr)
        sys.exit(2)
    if args.op == "models":
        models_mode(args)  # the parent starts one child per shape and never touches the GPU
        return
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    if args.mode == "copy":
        copy_mode(args)
        return
    if args.mode == "stamps":
        (mla_stamps_mode if args.op == "mla" else stamps_mode)(args)
        return
    if args.mode == "read":
        read_mode(args)
        return
    if args.op == "kv_append":
        kv_append_mode(args)
        return
    if args.op == "mla":
        mla_mode(args)
        return
    if args.op == "sweep":
        sweep_mode(args)
        return
    if args.op == "splits":
        splits_mode(args)
        return

    import attention_amd
    from attention_amd import cabi
    from attention_amd.cases import algorithmic_bytes, algorithmic_flops, get_config

    if not attention_amd.is_cuda_extension_loaded():
        raise RuntimeError("HIP op library not loaded; run __graft_entry__.build()")
    cfg = get_config(args.config)
    dev = torch.device("cuda:0")
    t0 = time.perf_counter()
    lengths = cfg.lengths()
    if args.device_gen:
        case = cfg.make(device=dev, device_gen=True, lengths=lengths)
        case_cpu = None
    else:
        case_cpu = cfg.make(device="cpu", lengths=lengths)
        case = tuple(x.to(dev) for x in case_cpu)
    q, k, v, table, lens = case
    kv_bytes = 2 * k.numel() * k.element_size()
    pools = args.pools or max(2, math.ceil(768e6 / kv_bytes))
    ks, vs = [k], [v]
    for i in range(1, pools):
        ks.append(k.roll(i, dims=0).contiguous())
        vs.append(v.roll(i, dims=0).contiguous())
    torch.cuda.synchronize()
    log(f"{cfg.name}: {len(lengths)} seqs, sum len {sum(lengths)}, KV pool {kv_bytes / 1e6:.1f} MB "
        f"x {pools} pools, setup {time.perf_counter() - t0:.1f}s")

    elem = q.element_size()
    alg_bytes = algorithmic_bytes(lengths, cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim,
                                  cfg.block_size, elem)
    scale = 1.0 / math.sqrt(cfg.head_dim)
    stream = torch.cuda.current_stream(dev)
    auto_kind, auto_waves, splits, chunk = cabi.auto_info(cfg.batch, cfg.q_heads, cfg.kv_heads,
                                                          cfg.head_dim, cfg.block_size, table.shape[1],
                                                          cabi.DTYPE[q.dtype])

    valu_stage = cabi.QD_STAGE_VALU if args.compute == "valu" else 0
    if args.compute == "valu":
        if args.kernel != "auto" or args.splits:
            raise SystemExit("--compute valu applies to the automatic balanced path only")
        path = "C ABI qd_gqa_decode_auto_stages with QD_STAGE_VALU (VALU math, comparison)"
        vws = torch.empty(cabi.auto_workspace_bytes(cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim,
                                                    cfg.block_size, table.shape[1], cabi.DTYPE[q.dtype]),
                          device=dev, dtype=torch.uint8)
        vout = torch.empty_like(q)

        def step(i):
            rc = cabi.auto_launch(q, ks[i % pools], vs[i % pools], table, lens, vout, scale=scale, workspace=vws,
                                  stream=stream.cuda_stream, stages=cabi.QD_STAGE_ALL | valu_stage)
            if rc:
                raise RuntimeError(cabi.error_string(rc))
    elif args.kernel == "auto" and args.splits == 0:
        path = "torch.ops.qd_attention.gqa_decode (automatic path)"

        def step(i):
            attention_amd.gqa_decode(q, ks[i % pools], vs[i % pools], table, lens)
    else:
        if args.splits:
            splits, chunk = args.splits, args.chunk_pages
        flags = cabi.QD_FLAG_FORCE_GENERIC if args.kernel == "generic" else 0
        out = torch.empty_like(q)
        ws = torch.empty(max(1, cfg.batch * cfg.q_heads * splits * (cfg.head_dim + 2)), device=dev)
        path = f"C ABI qd_gqa_decode_launch kernel={args.kernel}"

        def step(i):
            rc = cabi.launch(q, ks[i % pools], vs[i % pools], table, lens, out, scale=scale,
                             splits=splits, chunk_pages=chunk, workspace=ws, flags=flags,
                             stream=stream.cuda_stream)
            if rc:
                raise RuntimeError(cabi.error_string(rc))
    kind = cabi.lib().qd_gqa_decode_kernel_kind(cfg.q_heads, cfg.kv_heads, cfg.head_dim,
                                                cfg.block_size, cabi.DTYPE[q.dtype],
                                                cabi.QD_FLAG_FORCE_GENERIC if args.kernel == "generic" else 0)
    if args.kernel == "auto" and args.splits == 0 and auto_kind == 1:
        kname, kernels = "decode_mfma_sk_kernel", "decode_mfma_sk_kernel+merge_sk_kernel"
    else:
        kname = "decode_mfma_kernel" if kind == 1 else "decode_generic_kernel"
        kernels = kname + ("+combine_kernel" if splits > 1 else "")
    log(f"path: {path}; kernels {kernels}; waves={auto_waves} splits={splits} chunk_pages={chunk}; "
        f"warmup {args.warmup}, {SAMPLES} samples of {args.steps} steps")
    call_ms = time_samples(step, args.steps, args.warmup, stream)
    ms = statistics.median(call_ms)
    us = ms * 1e3
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    log(f"{us:.2f} us/call (median of {SAMPLES} samples; min {min(call_ms) * 1e3:.2f}, max "
        f"{max(call_ms) * 1e3:.2f}), {gbs:.1f} GB/s algorithmic ({100 * gbs / PEAK_HBM_GBS:.1f}% of peak)")

    # Roofline of the dominant kernel alone: the decode stage of the same
    # call (qd_gqa_decode_auto_stages), timed with HIP events on its stream.
    if auto_kind == 1 and args.kernel == "auto" and args.splits == 0:
        rk_name = kname
        rws = torch.zeros(cabi.auto_workspace_bytes(cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim,
                                                    cfg.block_size, table.shape[1], cabi.DTYPE[q.dtype]),
                          device=dev, dtype=torch.uint8)
        rout = torch.empty_like(q)

        def decode_stage(i):
            rc = cabi.auto_launch(q, ks[i % pools], vs[i % pools], table, lens, rout, scale=scale,
                                  workspace=rws, stream=stream.cuda_stream, stages=cabi.QD_STAGE_DECODE | valu_stage)
            if rc:
                raise RuntimeError(cabi.error_string(rc))

        k_ms = statistics.median(time_samples(decode_stage, args.steps, args.warmup, stream))
        rk_note = ("achieved = algorithmic bytes per call / average duration of the decode kernel "
                   "alone (decode stage of qd_gqa_decode_auto_stages, HIP events on its stream, median of "
                   f"{SAMPLES} samples)")
    else:
        rk_name, k_ms = kernels, ms
        rk_note = "achieved = algorithmic bytes per call / HIP-event time per call (all launches)"
    k_gbs = alg_bytes / (k_ms * 1e-3) / 1e9
    log(f"{rk_name}: {k_ms * 1e3:.2f} us/launch, {k_gbs:.1f} GB/s ({100 * k_gbs / PEAK_HBM_GBS:.1f}% of peak)")
    traffic = profiled_traffic(rk_name, cfg.name)

    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "us_per_call": round(us, 3),
        "us_per_call_samples": [round(x * 1e3, 3) for x in call_ms],
        "us_per_call_min": round(min(call_ms) * 1e3, 3),
        "us_per_call_max": round(max(call_ms) * 1e3, 3),
        "pct_of_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
        "n_gpus": 1,
        "steps": args.steps,
        "samples": SAMPLES,
        "timing": (f"{args.warmup} warmup calls, then {SAMPLES} samples of {args.steps} calls each bracketed "
                   "by synchronizations and HIP events; value and ms_per_step are the median sample "
                   "(reference benchmarks/measure_decode.py:47-57)"),
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DT_NAME[q.dtype],
        "data": ("synthetic: seeded reference recipe (benchmarks/data.py:8-43), "
                 f"{'GPU' if args.device_gen else 'CPU'}-drawn N(0,1) q/K/V, shuffled exact pool"),
        "config": {
            "workload": f"{cfg.name}: {cfg.description}",
            "batch": cfg.batch, "q_heads": cfg.q_heads, "kv_heads": cfg.kv_heads,
            "head_dim": cfg.head_dim, "block_size": cfg.block_size,
            "context_lens": (list(cfg.fixed_lengths) if cfg.fixed_lengths else
                             f"U{list(cfg.len_range)} seed {10_000 + cfg.seed}: sum {sum(lengths)}, "
                             f"min {min(lengths)}, max {max(lengths)}"),
            "kv_pools_rotated": pools, "path": path, "kernels": kernels, "compute": args.compute,
            "waves": auto_waves if auto_kind == 1 else None, "splits": splits, "chunk_pages": chunk,
            "algorithmic_bytes_per_call": alg_bytes,
            "flops_per_call": algorithmic_flops(lengths, cfg.q_heads, cfg.head_dim),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": rk_name,
            "achieved": round(k_gbs, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(k_gbs / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "duration_us": round(k_ms * 1e3, 3),
            "algorithmic_bytes": alg_bytes,
            "note": rk_note + ("; traffic = calibrated FETCH_SIZE + WRITE_SIZE bytes per dispatch "
                               "from profiles/" if traffic else ""),
        },
    }
    if not args.no_cpu_baseline:
        if case_cpu is None:
            case_cpu = tuple(x.cpu() for x in case)
        log("timing the reference CPU path ...")
        result["cpu_baseline"] = cpu_baseline(case_cpu, cfg, args.cpu_repeats)
        cb = result["cpu_baseline"]
        log(f"cpu baseline {cb['value']} GB/s ({cb['us_per_call']} us/call) on {cb['cores']} threads "
            f"{cb['threads_from']}; cfg1 {cb['cfg1_us_per_call']} us/call")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
