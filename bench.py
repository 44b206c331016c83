"""Benchmark of the MI355X expert-paging hot path (one GPU).

Headline (the `value`): Huffman decode GB/s -- one step is one launch of the
batched row expansion over 256 synthetic experts (w13 fp8 1024x2048 + w2 fp8
2048x512, N(0, 0.02) weights quantised to e4m3 with 128x128 block scales,
compressed per row at pitch 0.89), inputs resident in HBM. Bytes per row
= 4(G+1) + N/2 + 4*gstart[G] + 512 + N (header, nibbles, Huffman words
consumed, LUT, raw output). Also reported: slot gather GB/s from pinned host
RAM against the in-run host-link ceiling (large pinned H2D copies), acquire
microseconds per layer inside a captured hipGraph, and the oracle's CPU
decoder on a bounded sample as the CPU baseline.

    python bench.py [--gpus 1] [--steps 200] [--warmup 50]
"""

import argparse
import concurrent.futures as cf
import ctypes
import json
import mmap
import os
import shutil
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "vllm-expert-pager_amd"))

import numpy as np  # noqa: E402
import torch  # noqa: E402

HBM_PEAK_GBPS = 8000.0
MFMA_FP8_PEAK_TFLOPS = 5000.0  # dense fp8 MFMA, MI355X
SHAPES = ((1024, 2048), (2048, 512))  # w13, w2 (rows, cols) of fp8
PITCH_RATIO = 0.89


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def synthetic_experts(count: int, seed: int, dev) -> list[torch.Tensor]:
    """fp8 e4m3 bytes of `count` experts per name, generated on the GPU: (count, N) uint8."""
    g = torch.Generator(device=dev).manual_seed(seed)
    out = []
    for r, c in SHAPES:
        rows = torch.empty((count, r * c), dtype=torch.uint8, device=dev)
        for j in range(count):
            w = torch.randn((r, c), generator=g, device=dev) * 0.02
            blk = w.view(r // 128, 128, c // 128, 128)
            s = blk.abs().amax(dim=(1, 3), keepdim=True).clamp(min=1e-12) / 448.0
            rows[j] = (blk / s).to(torch.float8_e4m3fn).view(torch.uint8).reshape(-1)
        out.append(rows)
    return out


def encode_batch(raws_host: list[np.ndarray], threads: int):
    from vllm_expert_pager import codec

    count = raws_host[0].shape[0]
    pitches = [codec.pitch_of(r.shape[1], PITCH_RATIO, 4096) for r in raws_host]
    stg = [np.empty((count, p), np.uint8) for p in pitches]
    luts = np.empty((count, len(raws_host), 512), np.uint8)

    def one(args):
        k, j = args
        codec.encode_into(raws_host[k][j], stg[k][j], luts[j, k])

    with cf.ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(one, [(k, j) for k in range(len(raws_host)) for j in range(count)]))
    return stg, luts


def algorithmic_bytes(stg: list[np.ndarray], n_bytes: list[int], chunk: int = 512) -> int:
    total = 0
    for k, s in enumerate(stg):
        n = n_bytes[k]
        G = n // (chunk * 32)
        words = s[:, 4 * G : 4 * G + 4].view(np.int32).astype(np.int64).reshape(-1)  # gstart[G]
        total += int(((4 * (G + 1) + n // 2 + 512 + n) * s.shape[0]) + 4 * words.sum())
    return total


def decode_traffic(rows: int):
    """HBM bytes per decode launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    scaled by the same counters on a plain device copy), read from the committed profile
    summary of the same workload; None when there is none for this row count."""
    path = os.path.join(ROOT, "profiles", f"decode_traffic_{rows}rows.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1])
    return None


# VALU issue model of one MI355X: 256 CUs x 4 SIMDs, one wave64 VALU instruction per SIMD
# every 4 clocks, 2.4 GHz peak engine clock.
SIMDS, VALU_CLOCKS, ENGINE_GHZ = 1024, 4, 2.4


def decode_valu(rows: int, alg_bytes: int, achieved_gbps: float, n_bytes: list[int], chunk: int = 512):
    """The decoder's VALU bound: VALU instructions per wave and symbol step (SQ_INSTS_VALU per
    dispatch / waves / steps, from the committed rocprofv3 --pmc summary of the same launch),
    the launch time that many instructions take on every SIMD at the peak clock, the
    algorithmic GB/s that allows, and the measured rate as a fraction of it; None when there
    is no summary for this row count."""
    path = os.path.join(ROOT, "profiles", f"decode_pmc_{rows}rows.md")
    if not os.path.exists(path):
        return None
    per_step = None
    for line in open(path):
        if line.startswith("| SQ_INSTS_VALU |"):
            per_step = float(line.split("|")[3])
    if per_step is None:
        return None
    groups = sum(n // (chunk * 32) for n in n_bytes)
    waves = rows * groups / 2  # two 32-lane groups per wave
    ms = waves * chunk * per_step * VALU_CLOCKS / (SIMDS * ENGINE_GHZ * 1e9) * 1e3
    ceiling = alg_bytes / (ms * 1e-3) / 1e9
    return {"insts_per_wave_step": per_step, "symbols_per_wave_step": 64, "ms_at_peak_issue": round(ms, 4),
            "ceiling_gbps": round(ceiling, 1), "ceiling_frac_of_hbm": round(ceiling / HBM_PEAK_GBPS, 4),
            "frac": round(achieved_gbps / ceiling, 4),
            "model": f"{SIMDS} SIMDs, one wave64 VALU instruction per {VALU_CLOCKS} clocks, {ENGINE_GHZ} GHz",
            "source": f"profiles/decode_pmc_{rows}rows.md"}


def warm_by_time(step, min_ms: float = 200.0, batch: int = 10, tol: float = 0.02, max_s: float = 5.0) -> dict:
    """Launch `step` in batches until at least `min_ms` of launches have run and
    two consecutive batches agree within `tol`, so the timed launches that
    follow run at steady clocks whatever --warmup is (at most `max_s`)."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    spent, prev, batches = 0.0, None, 0
    t0 = time.time()
    while True:
        e0.record()
        for _ in range(batch):
            step()
        e1.record()
        e1.synchronize()
        ms = e0.elapsed_time(e1) / batch
        spent += ms * batch
        batches += 1
        steady = prev is not None and abs(ms - prev) <= tol * prev
        if (spent >= min_ms and steady) or time.time() - t0 > max_s:
            return {"launches": batches * batch, "ms": round(spent, 1), "steady": steady,
                    "last_ms_per_launch": round(ms, 4)}
        prev = ms


def bench_decode(args, dev, cores):
    from oracle import codec_ref
    from vllm_expert_pager import codec

    count = args.rows
    t0 = time.time()
    raws = synthetic_experts(count, 1234, dev)
    raws_host = [r.cpu().numpy() for r in raws]
    stg_np, luts_np = encode_batch(raws_host, threads=max(1, min(16, cores)))
    log(f"prepared {count} experts in {time.time() - t0:.1f}s")
    n_bytes = [r.shape[1] for r in raws_host]
    stg = [torch.from_numpy(s).to(dev) for s in stg_np]
    lut = torch.from_numpy(luts_np).to(dev)
    dst = [torch.zeros_like(r) for r in raws]
    todo = torch.arange(count, dtype=torch.int64, device=dev)
    dst_row = torch.arange(count, dtype=torch.int64, device=dev)
    no_cache = torch.full((count,), -1, dtype=torch.int64, device=dev)
    alg = algorithmic_bytes(stg_np, n_bytes)

    def step():
        codec.decode_rows(todo, dst_row, no_cache, stg, dst, lut)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    warm = warm_by_time(step)
    log(f"decode warm-up: {warm}")
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    ok = all(torch.equal(d, r) for d, r in zip(dst, raws))
    if not ok:
        raise SystemExit("decode output differs from the raw rows")
    gbps = alg / (ms * 1e-3) / 1e9
    raw_gbps = sum(n_bytes) * count / (ms * 1e-3) / 1e9
    log(f"decode: {ms:.3f} ms/launch, {gbps:.1f} GB/s algorithmic, {raw_gbps:.1f} GB/s raw output")

    # Sweep of rows per launch (1..256): same kernel, shorter todo. A decode
    # step expands the misses of one layer, about 1-2 rows per launch.
    sweep, sweep_us = {}, {}
    for r in (1, 2, 4, 8, 32, 64, 128):
        if r >= count:
            continue
        t = todo[:r]
        for _ in range(2):
            codec.decode_rows(t, dst_row, no_cache, stg, dst, lut)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(5):
            codec.decode_rows(t, dst_row, no_cache, stg, dst, lut)
        e1.record()
        torch.cuda.synchronize()
        ms_r = e0.elapsed_time(e1) / 5
        sweep[str(r)] = round(algorithmic_bytes([s[:r] for s in stg_np], n_bytes) / (ms_r * 1e-3) / 1e9, 1)
        sweep_us[str(r)] = round(ms_r * 1e3, 1)
    sweep[str(count)] = round(gbps, 1)
    sweep_us[str(count)] = round(ms * 1e3, 1)

    # The same rows read straight from pinned RAM (xp_decode_rows_from_ram, the decode step's
    # path for compressed misses): 1-8 experts per launch, records read over the host link while
    # they are expanded, scale rows copied alongside; checked against the raw rows.
    from vllm_expert_pager.gather import DeviceRows
    from vllm_expert_pager.store import PinnedBuffer

    nr = min(8, count)
    bufs = [PinnedBuffer(nr * s.shape[1], coherent=False) for s in stg_np]
    hosts = [b.tensor(torch.uint8, (nr, s.shape[1])) for b, s in zip(bufs, stg_np)]
    for h, s in zip(hosts, stg_np):
        h.copy_(torch.from_numpy(s[:nr]))
    ram = [DeviceRows(h, b.device_ptr) for h, b in zip(hosts, bufs)]
    src_row = torch.arange(count, dtype=torch.int64, device=dev)
    scale = [torch.arange(count * 32, dtype=torch.int32, device=dev).view(count, 32) for _ in stg_np]
    scale_dst = [torch.zeros((count, 32), dtype=torch.int32, device=dev) for _ in stg_np]
    ram_us = {}
    for r in (1, 2, 4, 8):
        if r > nr:
            continue
        for d in dst:
            d[:r].zero_()
        t = todo[:r]
        args_r = (t, dst_row, no_cache, src_row, 0, ram, dst, lut, scale, scale_dst)
        codec.decode_rows_from_ram(*args_r)
        torch.cuda.synchronize()
        if not all(torch.equal(d[:r], w[:r]) for d, w in zip(dst, raws)):
            raise SystemExit("decode from the RAM tier differs from the raw rows")
        e0.record()
        for _ in range(5):
            codec.decode_rows_from_ram(*args_r)
        e1.record()
        torch.cuda.synchronize()
        ram_us[str(r)] = round(e0.elapsed_time(e1) / 5 * 1e3, 1)
    del ram, hosts
    for b in bufs:
        b.free()
    log(f"decode from pinned RAM, us by rows: {ram_us}")

    # CPU baseline: the oracle's C decoder on a bounded sample, all cores.
    sample = max(1, min(args.cpu_rows, count))
    t0 = time.perf_counter()
    reps = 0
    while True:
        for k in range(len(stg_np)):
            out = codec_ref.decode_fast(stg_np[k][:sample], luts_np[:sample, k], n_bytes[k], threads=cores)
            assert np.array_equal(out, raws_host[k][:sample])
        reps += 1
        if time.perf_counter() - t0 > args.cpu_seconds:
            break
    cpu_s = (time.perf_counter() - t0) / reps
    cpu_gbps = algorithmic_bytes([s[:sample] for s in stg_np], n_bytes) / cpu_s / 1e9
    log(f"cpu decode: {cpu_gbps:.2f} GB/s on {cores} threads ({sample} experts x {reps} reps)")
    return {
        "ms": ms,
        "warm": warm,
        "gbps": gbps,
        "raw_gbps": raw_gbps,
        "alg_bytes": alg,
        "n_bytes": n_bytes,
        "sweep": sweep,
        "sweep_us": sweep_us,
        "ram_us": ram_us,
        "cpu": {"value": round(cpu_gbps, 3), "unit": "GB/s", "cores": cores, "kind": "port",
                "sample": f"oracle C decoder (the reference's sequential decode rule), {sample} of the "
                          f"{count} experts (w13+w2 rows), {reps} repetitions, threads over groups"},
    }


def bench_encode(args, dev, cores):
    """GPU encoder (load time) over the synthetic experts of the decode leg, against the host
    encoder on the host's cores; records checked byte for byte against the host on a sample."""
    from vllm_expert_pager import codec

    count = args.rows
    raws = synthetic_experts(count, 4321, dev)
    pitches = [codec.pitch_of(r.shape[1], PITCH_RATIO, 4096) for r in raws]
    outs = [codec.encode_rows(r, p) for r, p in zip(raws, pitches)]
    torch.cuda.synchronize()

    def step():
        for r, p, (rec, lut, _) in zip(raws, pitches, outs):
            codec.encode_rows(r, p, records=rec, luts=lut, check=False)

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    steps = max(1, args.steps // 4)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    raw_bytes = count * sum(r.shape[1] for r in raws)
    out_bytes = sum(int(o[2].sum().item()) + count * codec.LUT_BYTES for o in outs)
    # byte parity on a sample against the host encoder
    sample = [0, count // 2, count - 1]
    ok = True
    for k, r in enumerate(raws):
        host = r[sample].cpu().numpy()
        for i, j in enumerate(sample):
            rec = np.empty(pitches[k], np.uint8)
            lut = np.empty(codec.LUT_BYTES, np.uint8)
            codec.encode_into(host[i], rec, lut)
            ok = ok and np.array_equal(outs[k][0][j].cpu().numpy(), rec) and np.array_equal(outs[k][1][j].cpu().numpy(), lut)
    # CPU baseline: the host encoder over a sample of experts, all cores.
    n_cpu = max(1, min(args.cpu_rows, count))
    hosts = [r[:n_cpu].cpu().numpy() for r in raws]
    reps, t0 = 0, time.perf_counter()
    while True:
        encode_batch(hosts, threads=max(1, cores))
        reps += 1
        if time.perf_counter() - t0 > args.cpu_seconds / 4:
            break
    cpu_s = (time.perf_counter() - t0) / reps
    cpu_gbps = n_cpu * sum(r.shape[1] for r in raws) / cpu_s / 1e9
    out = {
        "workload": f"encode {count} experts (w13 fp8 1024x2048 + w2 fp8 2048x512 rows, block-scaled N(0,0.02)) "
                    "at pitch 0.89, one launch per name",
        "ms": round(ms, 4),
        "raw_gbps": round(raw_bytes / (ms * 1e-3) / 1e9, 2),
        "hbm_gbps": round((raw_bytes + out_bytes) / (ms * 1e-3) / 1e9, 2),
        "hbm_frac": round((raw_bytes + out_bytes) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "bit_exact_sample": ok,
        "cpu_baseline": {"value": round(cpu_gbps, 3), "unit": "GB/s of raw rows", "cores": cores, "kind": "port",
                         "sample": f"host encoder (the reference's encode rule in C++), {n_cpu} experts x "
                                   f"{reps} repetitions, threads over rows"},
    }
    log(f"encode: {out}")
    return out


def bench_gather(args, dev):
    """Slot gather from pinned host RAM vs the in-run host-link ceiling."""
    from vllm_expert_pager import gather
    from vllm_expert_pager.store import PinnedBuffer

    n_bytes = [r * c for r, c in SHAPES]
    rows = 64
    K = 32
    out = {}
    for coherent in (True, False):
        bufs = [PinnedBuffer(rows * n, coherent) for n in n_bytes]
        host = [b.tensor(torch.uint8, (rows, n)) for b, n in zip(bufs, n_bytes)]
        for h in host:
            h.copy_(torch.randint(0, 256, h.shape, dtype=torch.uint8))
        from vllm_expert_pager.gather import DeviceRows

        src = [DeviceRows(h, b.device_ptr) for h, b in zip(host, bufs)]
        dst = [torch.empty((K, n), dtype=torch.uint8, device=dev) for n in n_bytes]
        scale = [torch.zeros((rows, 16), dtype=torch.int32, device=dev) for _ in n_bytes]
        sdst = [torch.zeros((K, 16), dtype=torch.int32, device=dev) for _ in n_bytes]
        todo = torch.arange(K, dtype=torch.int64, device=dev)
        dst_row = torch.arange(rows, dtype=torch.int64, device=dev) % K
        no_cache = torch.full((rows,), -1, dtype=torch.int64, device=dev)
        src_row = torch.arange(rows, dtype=torch.int64, device=dev)
        total = K * sum(n_bytes)

        def run():
            gather.gather_rows(todo, dst_row, no_cache, src_row, 0, src, dst, dst, None, scale, sdst)

        for _ in range(2):
            run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.gather_steps):
            run()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.gather_steps
        ok = all(torch.equal(dst[k].cpu(), host[k][:K]) for k in range(2))
        # Host-link ceiling: the copy engine moving the same bytes, best of several.
        best = 0.0
        for _ in range(5):
            e0.record()
            for k in range(2):
                dst[k].copy_(host[k][:K], non_blocking=True)
            e1.record()
            torch.cuda.synchronize()
            best = max(best, total / (e0.elapsed_time(e1) * 1e-3) / 1e9)
        key = "fine" if coherent else "coarse"
        out[key] = {"gbps": round(total / (ms * 1e-3) / 1e9, 2), "ceiling_gbps": round(best, 2), "ok": ok}
        log(f"gather ({key}-grained pinned): {out[key]}")
        if coherent:
            # CPU baseline: the same K rows memcpy'd from the pinned tier into
            # a host buffer by the host's cores (threads over 1 MiB pieces).
            cores = len(os.sched_getaffinity(0))
            src_np = [h[:K].numpy().reshape(-1) for h in host]
            dst_np = [np.empty_like(a) for a in src_np]
            piece = 1 << 20
            jobs = [(k, o) for k in range(2) for o in range(0, src_np[k].size, piece)]

            def cp(job):
                k, o = job
                np.copyto(dst_np[k][o : o + piece], src_np[k][o : o + piece])

            with cf.ThreadPoolExecutor(cores) as pool:
                list(pool.map(cp, jobs))
                reps, t0 = 0, time.perf_counter()
                while time.perf_counter() - t0 < args.cpu_seconds / 4:
                    list(pool.map(cp, jobs))
                    reps += 1
            cpu = total * reps / (time.perf_counter() - t0) / 1e9
            out["cpu_baseline"] = {"value": round(cpu, 2), "unit": "GB/s", "cores": cores, "kind": "port",
                                   "sample": f"memcpy of the same {K} rows from pinned RAM to a host buffer, "
                                             f"{reps} repetitions"}
            log(f"cpu gather: {cpu:.1f} GB/s on {cores} threads")
        for b in bufs:
            b.free()
    return out


def bench_acquire(args, dev):
    """Acquire of both tables for 40 layers inside one captured hipGraph."""
    from vllm_expert_pager.acquire import AcquirePair
    from vllm_expert_pager.table import ExpertTable

    L, E, S, R = 40, 256, 32, 256
    pairs = []
    for _ in range(L):
        v, r = ExpertTable(E, S, dev), ExpertTable(E, R, dev)
        r.slot_of[:R] = r.experts[:R]
        r.expert_in[:R] = r.experts[:R]
        pairs.append(AcquirePair(v, r))
    ids = torch.zeros((L, 1, 8), dtype=torch.int32, device=dev)
    rng = np.random.default_rng(5)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for layer in range(L):
            pairs[layer](ids[layer])
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for layer in range(L):
                pairs[layer](ids[layer])
    torch.cuda.synchronize()
    perm = rng.permutation(E)
    p = np.arange(1, E + 1, dtype=np.float64) ** -1.1
    p /= p.sum()
    steps = 50
    host_ids = np.stack([[perm[rng.choice(E, 8, replace=False, p=p)] for _ in range(L)] for _ in range(steps)])
    dev_ids = torch.from_numpy(host_ids.astype(np.int32)).to(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for i in range(3):
        ids.copy_(dev_ids[i].view(L, 1, 8))
        g.replay()
    torch.cuda.synchronize()
    total = 0.0
    for i in range(steps):
        ids.copy_(dev_ids[i].view(L, 1, 8))
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        total += e0.elapsed_time(e1)
    us_layer = total / steps / L * 1e3
    log(f"acquire: {us_layer:.2f} us/layer (graph of {L} layers, both tables)")
    # CPU baseline: the oracle's numpy restatement of ExpertTable.acquire
    # (table.py:75-128) on the same routing, both tables per layer: one thread,
    # then every core, as independent processes that each own a share of the
    # layers (a decode step runs its layers in order, so the all-cores figure
    # is a throughput no single step could reach).
    import subprocess
    import tempfile

    from oracle.table_ref import acquire_trace_rate

    n1, dt1 = acquire_trace_rate(host_ids, E, S, R, args.cpu_seconds / 4)
    cpu_us = dt1 / n1 * 1e6
    log(f"cpu acquire: {cpu_us:.1f} us/layer, one thread ({n1 // L} steps x {L} layers)")
    workers = max(1, min(len(os.sched_getaffinity(0)), L, 16))
    seconds = args.cpu_seconds / 4
    with tempfile.TemporaryDirectory() as tmp:
        procs = []
        start_at = time.time() + 3.0  # after every child has imported numpy
        for w in range(workers):
            path = os.path.join(tmp, f"ids{w}.npy")
            np.save(path, np.ascontiguousarray(host_ids[:, w::workers]))
            procs.append(subprocess.Popen(
                [sys.executable, "-m", "oracle.table_ref", path, str(E), str(S), str(R), str(seconds),
                 repr(start_at)], cwd=ROOT, stdout=subprocess.PIPE, text=True,
                env={**os.environ, "OMP_NUM_THREADS": "1", "OPENBLAS_NUM_THREADS": "1"}))
        done = []
        for p in procs:
            out, _ = p.communicate(timeout=seconds + 120)
            if p.returncode:
                raise RuntimeError(f"acquire baseline worker failed ({p.returncode})")
            n, dt = out.split()
            done.append((int(n), float(dt)))
    rate = sum(n / dt for n, dt in done)  # layer acquires per second, all workers overlapped
    all_us = 1e6 / rate
    log(f"cpu acquire: {all_us:.2f} us/layer over {workers} processes")
    sample = f"oracle numpy acquire of both tables, the same Zipf routing of {L} layers"
    return {"us_per_layer": round(us_layer, 3),
            "cpu_baseline": {"value": round(cpu_us, 2), "unit": "us/layer", "cores": 1, "kind": "port",
                             "sample": f"{sample}, {n1 // L} steps on one thread"},
            "cpu_baseline_all_cores": {
                "value": round(all_us, 3), "unit": "us/layer", "cores": workers, "kind": "port",
                "sample": f"{sample}, {workers} processes over {seconds:.1f} s, each owning every "
                          f"{workers}th layer; us/layer = 1 / (summed layer acquires per second)"}}


def bench_moe(args, dev):
    """Expert FFN of one prefill layer: 2048 tokens x top-8 over 256 experts.

    Experts are w13 fp8 1024x2048 + w2 fp8 2048x512 with 128x128 block
    scales, tokens bf16 ~N(0,1), softmax gate weights over the top 8 of
    random logits (near-uniform coverage). Times the two GEMM launches over
    a 256-slot slab (one-shot), the whole layer (quantise, route, GEMMs,
    top-k sum), the overflow path's compute over four 64-row chunks,
    which must give the one-shot bits, and the batch-1 decode step of the
    same layer (two launches per step).
    """
    from vllm_expert_pager import moe

    E, H, I, T, topk, W = 256, 2048, 512, 2048, 8, 64
    g = torch.Generator(device=dev).manual_seed(7)

    def quantised(n, k):
        q = torch.empty((E, n, k), dtype=torch.uint8, device=dev)
        s = torch.empty((E, n // 128, k // 128), dtype=torch.float32, device=dev)
        for e in range(E):
            w = torch.randn((n, k), generator=g, device=dev) * 0.02
            b = w.view(n // 128, 128, k // 128, 128)
            se = (b.abs().amax(dim=(1, 3)) / 448.0).clamp_min(1e-10)
            q[e] = (b / se[:, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).view(n, k)
            s[e] = se
        return q, s

    w13, w13s = quantised(2 * I, H)
    w2, w2s = quantised(H, I)
    x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
    top, ids = torch.randn((T, E), generator=g, device=dev).topk(topk, dim=1)
    tw = torch.softmax(top, dim=1).float().contiguous()
    xq, xs = moe.quant_tokens(x)
    emap = torch.arange(E, dtype=torch.int32, device=dev)
    r = moe.route(ids, emap, E)
    contrib = torch.zeros((T * topk, H), dtype=torch.bfloat16, device=dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, reps):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    reps = max(3, args.moe_steps)
    ms_gemm = timed(lambda: moe.run_experts(xq, xs, tw, w13, w13s, w2, w2s, r, contrib), reps)
    one = moe.topk_sum(contrib, ids, E)
    ms_layer = timed(lambda: moe.fused_moe(x, tw, ids, w13, w13s, w2, w2s), reps)

    chunk_maps = []
    for k in range(E // W):
        m = torch.full((E,), -1, dtype=torch.int32, device=dev)
        m[k * W : (k + 1) * W] = torch.arange(W, dtype=torch.int32, device=dev)
        chunk_maps.append(m)
    contrib2 = torch.zeros_like(contrib)

    def chunked():
        xq2, xs2 = moe.quant_tokens(x)
        for k, m in enumerate(chunk_maps):
            rk = moe.route(ids, m, W)
            sl = slice(k * W, (k + 1) * W)
            moe.run_experts(xq2, xs2, tw, w13[sl], w13s[sl], w2[sl], w2s[sl], rk, contrib2)
        return moe.topk_sum(contrib2, ids, E)

    ms_chunked = timed(chunked, reps)
    two = chunked()
    exact = bool(torch.equal(one.view(torch.int16), two.view(torch.int16)))
    if not exact:
        raise SystemExit("chunked expert FFN differs from the one-shot run")
    # Batch-1 decode step of the same layer: one token, its top-8 experts
    # resident in the slab, the two-launch decode FFN. 64 steps with
    # different experts are captured in one graph so that launch overhead
    # and cache reuse of one expert set stay out of the figure.
    nd = 64
    x1 = torch.randn((nd, 1, H), generator=g, device=dev).to(torch.bfloat16)
    ids1 = torch.stack([torch.randperm(E, generator=g, device=dev)[:topk] for _ in range(nd)]).view(nd, 1, topk)
    tw1 = torch.softmax(torch.randn((nd, 1, topk), generator=g, device=dev), dim=2).contiguous()
    ids1 = ids1.to(torch.int64).contiguous()
    # Each step's pair slots, as the acquire kernel writes them for the pager.
    pslot1 = emap[ids1].contiguous()

    def decode_steps(pairs_from_acquire: bool):
        for i in range(nd):
            moe.decode_experts(x1[i], tw1[i], ids1[i], emap, E, w13, w13s, w2, w2s, E,
                               pair_slot=pslot1[i].view(-1) if pairs_from_acquire else None)

    us_decode = {}
    for mode in (True, False):
        decode_steps(mode)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            decode_steps(mode)
        us_decode[mode] = timed(graph.replay, reps) * 1e3 / nd
        del graph
    decode_bytes = topk * (2 * I * H + H * I)
    pairs = T * topk
    flops = 2.0 * pairs * (2 * I * H + H * I)
    weight_bytes = E * (2 * I * H + H * I) + 4 * (w13s.numel() + w2s.numel())
    # Minimum HBM traffic of the two GEMMs: weights once, tokens once, the
    # fp8 activation written and read, the bf16 contributions written.
    alg_bytes = weight_bytes + T * H + 4 * T * H // 128 + 2 * pairs * I + 2 * pairs * H
    tflops = flops / (ms_gemm * 1e-3) / 1e12
    out = {
        "workload": f"{T} tokens x top-{topk} over {E} experts (w13 2x{I}x{H}, w2 {H}x{I} fp8, 128x128 scales)",
        "ms_gemm": round(ms_gemm, 4),
        "tflops": round(tflops, 1),
        "mfma_frac": round(tflops / MFMA_FP8_PEAK_TFLOPS, 4),
        "hbm_gbps": round(alg_bytes / (ms_gemm * 1e-3) / 1e9, 1),
        "hbm_frac": round(alg_bytes / (ms_gemm * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "ms_layer_one_shot": round(ms_layer, 4),
        "ms_layer_chunked_4x64": round(ms_chunked, 4),
        "chunked_bit_exact": exact,
        "decode_ffn_batch1_us": round(us_decode[True], 2),
        "decode_ffn_batch1_weight_gbps": round(decode_bytes / (us_decode[True] * 1e-6) / 1e9, 1),
        "decode_ffn_batch1_us_ids_through_expert_map": round(us_decode[False], 2),
    }
    log(f"moe: {out}")
    return out


# ---- 40-layer decode trace with a Qwen3-MoE-shaped model ----

QWEN = {"layers": 40, "hidden": 2048, "heads": 32, "kv_heads": 4, "head_dim": 128, "experts": 256,
        "intermediate": 512, "topk": 8, "vocab": 151936, "rope_theta": 1e6, "eps": 1e-6}


def zipf_trace(rng, steps: int, layers: int, E: int, k: int, s: float, reuse: float) -> np.ndarray:
    """(steps, layers, k) expert ids: Zipf(s) over a per-layer permutation, k distinct per step;
    with probability `reuse` a layer repeats its previous step's set."""
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    perms = [rng.permutation(E) for _ in range(layers)]
    out = np.empty((steps, layers, k), np.int32)
    for t in range(steps):
        for l in range(layers):
            if t > 0 and rng.random() < reuse:
                out[t, l] = out[t - 1, l]
            else:
                out[t, l] = perms[l][rng.choice(E, k, replace=False, p=p)]
    return out


def quantised_experts(E: int, H: int, I: int, g, dev):
    """Synthetic block-fp8 experts on the GPU: N(0, 0.02) weights, one amax/448 scale per 128x128 block."""
    def one(n, k):
        q = torch.empty((E, n, k), dtype=torch.uint8, device=dev)
        s = torch.empty((E, n // 128, k // 128), dtype=torch.float32, device=dev)
        for e0 in range(0, E, 32):
            w = torch.randn((min(32, E - e0), n, k), generator=g, device=dev) * 0.02
            b = w.view(-1, n // 128, 128, k // 128, 128)
            se = (b.abs().amax(dim=(2, 4)) / 448.0).clamp_min(1e-10)
            q[e0 : e0 + w.shape[0]] = (b / se[:, :, None, :, None]).clamp(-448, 448).to(
                torch.float8_e4m3fn).view(torch.uint8).view(-1, n, k)
            s[e0 : e0 + w.shape[0]] = se
        return q, s
    w13, w13s = one(2 * I, H)
    w2, w2s = one(H, I)
    return w13, w13s, w2, w2s


class QwenMoeDecoder:
    """Random-init Qwen3-MoE-shaped decoder (bf16 non-expert weights) whose experts are paged.

    Per layer: RMSNorm, fused QKV projection, per-head q/k RMSNorm, rotary
    embedding, GQA attention over a static KV cache with a position mask,
    output projection added to the residual, RMSNorm, router (softmax over
    the logits of the traced ids), the paged expert FFN, residual. Final
    RMSNorm, LM head, greedy next token. Shapes are static, so one step is
    captured in a hipGraph; the non-expert part is written with few, fused
    torch launches (about 20 per layer).
    """

    def __init__(self, dev, pager, layers, trace, ctx: int):
        c = QWEN
        self.dev, self.pager, self.layers = dev, pager, layers
        H, nh, kv, hd = c["hidden"], c["heads"], c["kv_heads"], c["head_dim"]
        self.H, self.nh, self.kv, self.hd, self.ctx = H, nh, kv, hd, ctx
        g = torch.Generator(device=dev).manual_seed(11)
        bf = {"dtype": torch.bfloat16, "device": dev}
        rnd = lambda *shape: (torch.randn(shape, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        L = len(layers)
        self.w_qkv = [rnd((nh + 2 * kv) * hd, H) for _ in range(L)]
        self.w_o_t = [rnd(nh * hd, H) for _ in range(L)]        # output projection, stored (in, out)
        self.w_router = [rnd(c["experts"], H) for _ in range(L)]
        self.ln1 = [torch.ones(H, **bf) for _ in range(L)]
        self.ln2 = [torch.ones(H, **bf) for _ in range(L)]
        self.qkn = [torch.ones((nh + kv, hd), **bf) for _ in range(L)]  # q-norm rows, then k-norm rows
        self.embed = rnd(c["vocab"], H)
        self.lm_head = rnd(c["vocab"], H)
        self.norm = torch.ones(H, **bf)
        self.kcache = torch.zeros((L, kv, hd, ctx), **bf)   # K stored transposed: (kv, dim, ctx)
        self.vcache = torch.zeros((L, kv, ctx, hd), **bf)
        inv = 1.0 / (c["rope_theta"] ** (torch.arange(0, hd, 2, device=dev, dtype=torch.float32) / hd))
        ang = torch.arange(ctx, device=dev, dtype=torch.float32)[:, None] * inv[None, :]
        self.freqs = torch.polar(torch.ones_like(ang), ang)   # (ctx, hd/2) complex64
        self.trace = trace                                   # (steps, L, k) int32 on the device
        self.step = torch.zeros((1,), dtype=torch.int64, device=dev)
        self.pos = torch.zeros((1,), dtype=torch.int64, device=dev)
        self.token = torch.zeros((1,), dtype=torch.int64, device=dev)
        self.positions = torch.arange(ctx, device=dev)
        self.neg = torch.full((ctx,), float("-inf"), device=dev)
        self.zero = torch.zeros((ctx,), device=dev)

    def forward_step(self):
        F = torch.nn.functional
        nh, kv, hd, H, eps = self.nh, self.kv, self.hd, self.H, QWEN["eps"]
        ids_all = self.trace.index_select(0, self.step).squeeze(0).long()  # (L, k)
        h = self.embed.index_select(0, self.token)                         # (1, H)
        freqs = self.freqs.index_select(0, self.pos)                        # (1, hd/2)
        bias = torch.where(self.positions <= self.pos, self.zero, self.neg)  # attention mask for this step
        scale = hd ** -0.5
        for l, layer in enumerate(self.layers):
            x = F.rms_norm(h, (H,), self.ln1[l], eps)
            qkv = F.linear(x, self.w_qkv[l])[0]
            qk = F.rms_norm(qkv[: (nh + kv) * hd].view(nh + kv, hd), (hd,), None, eps) * self.qkn[l]
            qk = torch.view_as_real(torch.view_as_complex(qk.float().view(nh + kv, hd // 2, 2)) * freqs)
            qk = qk.reshape(nh + kv, hd).to(torch.bfloat16)
            v = qkv[(nh + kv) * hd :].view(kv, hd)
            self.kcache[l].index_copy_(2, self.pos, qk[nh:].unsqueeze(2))
            self.vcache[l].index_copy_(1, self.pos, v.unsqueeze(1))
            scores = torch.matmul(qk[:nh].view(kv, nh // kv, hd), self.kcache[l])  # (kv, g, ctx)
            probs = torch.softmax(torch.add(bias, scores, alpha=scale), dim=-1).to(torch.bfloat16)
            attn = torch.matmul(probs, self.vcache[l]).view(1, nh * hd)
            h = torch.addmm(h, attn, self.w_o_t[l])
            x2 = F.rms_norm(h, (H,), self.ln2[l], eps)
            ids = ids_all[l : l + 1]                                        # (1, k) traced routing
            w = torch.softmax(F.linear(x2, self.w_router[l]).gather(1, ids).float(), dim=-1)
            h = h + layer.forward(x2, w, ids)
        logits = F.linear(F.rms_norm(h, (H,), self.norm, eps), self.lm_head)
        # Greedy token in two single-workgroup reductions (vocab = 1187 x 128).
        best, idx = logits.view(-1, 128).max(dim=1)
        row = best.argmax().view(1)
        self.token.copy_((row * 128 + idx.index_select(0, row)).clamp_(0, QWEN["vocab"] - 1))
        self.pos.add_(1)
        self.step.add_(1)


def build_paged_model(dev, settings, keep_weights: bool = False):
    """The 40 MoE layers of 256 synthetic block-fp8 experts behind one pager (per-layer seeds)."""
    from vllm_expert_pager import pager as pg

    c = QWEN
    L, E, H, I = c["layers"], c["experts"], c["hidden"], c["intermediate"]
    t0 = time.time()
    pager = pg.Pager(settings, L, E, H, I, dev)
    layers, weights = [], []
    for l in range(L):
        g = torch.Generator(device=dev).manual_seed(1000 + l)
        layer = pager.add_layer()
        w13, w13s, w2, w2s = quantised_experts(E, H, I, g, dev)
        pager.store.write_rows(layer.layer, "w13_weight", w13.view(E, -1))
        pager.store.write_rows(layer.layer, "w2_weight", w2.view(E, -1))
        layer.setup({pg.SCALES[0]: w13s, pg.SCALES[1]: w2s})
        layers.append(layer)
        if keep_weights:
            weights.append((w13, w13s, w2, w2s))
        del w13, w2
        if (l + 1) % 10 == 0:
            log(f"model: {l + 1}/{L} layers written ({time.time() - t0:.1f}s)")
    torch.cuda.synchronize()
    st = pager.store
    log(f"model: {L} layers x {E} experts loaded in {time.time() - t0:.1f}s (RAM tier "
        f"{st.rows * st.record_bytes / 2**30:.1f} GiB pinned, {'compressed' if st.compress else 'raw'}"
        f"{', paging file ' + st.path if st.path else ''})")
    return pager, layers, weights


def decode_trace(args, dev, pager, layers, label: str, steps: int | None = None,
                 paging_steps: int | None = None) -> dict:
    """Run the Zipf(1.1)/0.7-reuse decode trace through a captured 40-layer step; tok/s, hit rates,
    and the paging path alone per layer (over `paging_steps` steps of a second trace, by default
    as many as the first)."""
    c = QWEN
    L, E, H, k = c["layers"], c["experts"], c["hidden"], c["topk"]
    steps, warm = steps or args.decode_steps, args.decode_warmup
    store = pager.store
    rng = np.random.default_rng(2025)
    trace = torch.from_numpy(zipf_trace(rng, warm + steps, L, E, k, 1.1, 0.7)).to(dev)
    model = QwenMoeDecoder(dev, pager, layers, trace, ctx=warm + steps + 1)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        model.forward_step()  # eager step 0 (also warms the allocator)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            model.forward_step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    # Capture records without running; replays continue from step 1.
    for _ in range(max(0, warm - 1)):
        graph.replay()
    torch.cuda.synchronize()
    before = [lay.hit_rates() for lay in layers]
    ssd0 = (store.fetches, store.reads, store.io_seconds) if store.path else None
    ph0 = store.phase_stats() if store.path else None
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    after = [lay.hit_rates() for lay in layers]
    d = [sum(a[i] - b[i] for a, b in zip(after, before)) for i in range(4)]
    ssd = None
    if ssd0 is not None:
        ssd = {"fetches": store.fetches - ssd0[0], "reads": store.reads - ssd0[1],
               "io_seconds": round(store.io_seconds - ssd0[2], 4), "failed": store.failed,
               "phases": _phase_delta(store.phase_stats(), ph0)}
    # The paging path alone on a continuing trace: acquire, gather (+ SSD
    # fetch, expansion), expert FFN and top-k sum of the 40 layers in one graph.
    x = torch.randn((1, H), device=dev).to(torch.bfloat16)
    wk = torch.full((1, k), 1.0 / k, device=dev)
    pstep = torch.zeros((1,), dtype=torch.int64, device=dev)
    ptrace = torch.from_numpy(zipf_trace(np.random.default_rng(7), warm + steps, L, E, k, 1.1, 0.7)).to(dev)

    def pager_step():
        ids_all = ptrace.index_select(0, pstep).squeeze(0).long()
        for l, layer in enumerate(layers):
            layer.forward(x, wk, ids_all[l : l + 1])
        pstep.add_(1)

    with torch.cuda.stream(s):
        pager_step()
        pgraph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(pgraph, stream=s):
            pager_step()
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(max(0, warm - 1)):
        pgraph.replay()
    torch.cuda.synchronize()
    psteps = paging_steps or steps
    e0.record()
    for _ in range(psteps):
        pgraph.replay()
    e1.record()
    torch.cuda.synchronize()
    pager_ms = e0.elapsed_time(e1) / psteps
    out = {
        "workload": label,
        "tok_s": round(1e3 / ms, 2),
        "ms_per_token": round(ms, 4),
        "us_per_layer": round(ms * 1e3 / L, 2),
        "vram_hit_rate": round(d[0] / max(1, d[0] + d[1]), 4),
        "ram_hit_rate": round(d[2] / max(1, d[2] + d[3]), 4),
        "misses_per_layer_step": round(d[1] / (L * steps), 3),
        "paging_path_us_per_layer": round(pager_ms * 1e3 / L, 2),
        "steps": steps,
    }
    if psteps != steps:
        out["paging_path_steps"] = psteps
    if ssd is not None:
        out["ssd"] = ssd
    log(f"decode trace: {out}")
    return out


def bench_model_decode(args, dev):
    """Decode trace: 40 MoE layers x 256 experts x 3 MiB, 32 cache slots, every expert in a raw pinned
    RAM tier, batch 1, top-8, Zipf(1.1) routing with 70% reuse of the previous step's set per layer.
    One decode step of the whole model is one hipGraph replay."""
    from vllm_expert_pager import pager as pg

    settings = pg.Settings(cache_slots=32, ram_slots=None, compress="off", working_rows=64, log_interval=0)
    pager, layers, _ = build_paged_model(dev, settings)
    try:
        return decode_trace(args, dev, pager, layers,
                            "40-layer decode trace, 256 experts x 3 MiB, 32 cache slots, all experts in a raw "
                            f"pinned RAM tier, batch 1, top-8, Zipf(1.1) with 0.7 reuse, {args.decode_steps} "
                            "steps in one captured hipGraph per step")
    finally:
        pager.close()


def bench_model_decode_compressed(args, dev):
    """The decode trace of bench_model_decode with every expert in a compressed RAM tier (pitch
    0.89, no paging file): each miss's record is expanded straight from pinned RAM by the decoder,
    with no copy to staging first. A quarter of the raw trace's steps."""
    from vllm_expert_pager import pager as pg

    settings = pg.Settings(cache_slots=32, ram_slots=None, compress="on", working_rows=64, log_interval=0)
    pager, layers, _ = build_paged_model(dev, settings)
    steps = max(100, args.decode_steps // 4)
    try:
        return decode_trace(args, dev, pager, layers,
                            "40-layer decode trace, 256 experts x 3 MiB, 32 cache slots, all experts in a RAM "
                            "tier of rows compressed at pitch 0.89 (expanded straight from pinned RAM), batch 1, "
                            f"top-8, Zipf(1.1) with 0.7 reuse, {steps} steps in one captured hipGraph per step",
                            steps=steps)
    finally:
        pager.close()


def disk_ceiling(path: str, record_bytes: int, records: int, seconds: float = 0.5) -> dict:
    """Record-sized O_DIRECT reads of the paging file at 1, 2, 4, 8 and 32 in flight, from a thread
    pool (the SSD server's way) and from io_uring: the disk's ceiling in this run."""
    from vllm_expert_pager import _native

    lib = _native.lib()
    fd = os.open(path, os.O_RDONLY | os.O_DIRECT)
    out = {"record_bytes": record_bytes}
    rng = np.random.default_rng(11)
    runs = {}
    try:
        # Two passes in different orders; each configuration keeps its better pass (a disk that
        # has just been written can serve some reads from its own cache).
        for order in ((8, 32, 4, 2, 1), (1, 2, 4, 32, 8)):
            for mode, name in ((0, "threads"), (1, "io_uring")):
                for depth in order:
                    # about `seconds` of reads at 3 GB/s, at least 4 per reader
                    count = max(4 * depth, int(3e9 * seconds / record_bytes))
                    idx = rng.choice(records, size=count, replace=count > records)
                    offs = (ctypes.c_int64 * count)(*(int(i) * record_bytes for i in idx))
                    sec = ctypes.c_double()
                    rc = lib.xp_ssd_read_probe(fd, record_bytes, offs, count, depth, mode, ctypes.byref(sec))
                    key = (name, str(depth))
                    if rc:
                        runs.setdefault(key, []).append(f"failed: {lib.xp_last_error().decode(errors='replace')}")
                    else:
                        runs.setdefault(key, []).append(round(count * record_bytes / sec.value / 1e9, 3))
    finally:
        os.close(fd)
    for (name, depth), vals in runs.items():
        nums = [v for v in vals if isinstance(v, float)]
        out.setdefault(f"{name}_gbps", {})[depth] = max(nums) if nums else vals[-1]
        out.setdefault(f"{name}_passes", {})[depth] = vals
    log(f"disk ceiling: {out}")
    return out


def disk_ceiling_loaded(path: str, record_bytes: int, records: int, dev, depths=(1, 2, 4, 8),
                        seconds: float = 0.5) -> dict:
    """The same thread-pool probe while the GPU streams pinned host memory (host-to-device copies
    of 1 GiB on a side stream, as a prefill chunk or decode step streams RAM-tier records while
    the server reads): the disk's ceiling under the workload's own host-link traffic. Two passes
    per depth, the better kept; the copy rate is reported beside it."""
    import threading

    from vllm_expert_pager import _native

    lib = _native.lib()
    src = torch.empty((1 << 30,), dtype=torch.uint8).pin_memory()
    dst = torch.empty((1 << 30,), dtype=torch.uint8, device=dev)
    stop = threading.Event()
    moved = [0, 0.0]

    def stream():
        s = torch.cuda.Stream(device=dev)
        t0 = time.perf_counter()
        with torch.cuda.stream(s):
            while not stop.is_set():
                for _ in range(4):
                    dst.copy_(src, non_blocking=True)
                s.synchronize()
                moved[0] += 4 * src.numel()
        moved[1] = time.perf_counter() - t0

    rng = np.random.default_rng(13)
    fd = os.open(path, os.O_RDONLY | os.O_DIRECT)
    out = {"threads_gbps": {}, "passes": {}}
    th = threading.Thread(target=stream)
    th.start()
    try:
        time.sleep(0.2)
        for order in (depths, depths[::-1]):
            for depth in order:
                count = max(4 * depth, int(3e9 * seconds / record_bytes))
                idx = rng.choice(records, size=count, replace=count > records)
                offs = (ctypes.c_int64 * count)(*(int(i) * record_bytes for i in idx))
                sec = ctypes.c_double()
                if lib.xp_ssd_read_probe(fd, record_bytes, offs, count, depth, 0, ctypes.byref(sec)):
                    out["passes"].setdefault(str(depth), []).append("failed")
                    continue
                out["passes"].setdefault(str(depth), []).append(round(count * record_bytes / sec.value / 1e9, 3))
    finally:
        stop.set()
        th.join()
        os.close(fd)
    for depth, vals in out["passes"].items():
        nums = [v for v in vals if isinstance(v, float)]
        out["threads_gbps"][depth] = max(nums) if nums else None
    out["h2d_gbps_alongside"] = round(moved[0] / moved[1] / 1e9, 1) if moved[1] > 0 else None
    del src, dst
    log(f"disk ceiling under host-link load: {out}")
    return out


def _phase_delta(after: dict, before: dict) -> dict:
    out = {k: round(after[k] - before.get(k, 0), 4) for k in ("busy_s", "queue_s", "read_s", "copy_s", "preads")}
    out.update(readers=after["readers"], bounce=after["bounce"])
    return out


def server_sweep(store, path: str, readers=(1, 2, 4, 8), seconds: float = 0.6) -> dict:
    """The SSD server alone, driven from the host: a second server instance on the paging file and
    the pinned RAM tier, at several reader counts, for requests of 8 random records (the size of a
    prefill chunk's SSD listing; two kept outstanding, as chunks are published one ahead) and of
    one record (a decode step's miss, one at a time). It writes only the working rows."""
    from vllm_expert_pager import _native

    lib = _native.lib()
    names = store.names
    n, rb = len(names), store.record_bytes
    ring, block = 4, 16
    slot_words = 2 + 2 * block
    records = store.num_layers * store.num_experts
    rng = np.random.default_rng(19)

    def aligned(count):
        raw = np.zeros(count + 512, np.int64)
        off = (-raw.ctypes.data % 4096) // 8
        return raw[off : off + count]

    out = {"record_bytes": rb, "readers": {}}
    fd = os.open(path, os.O_RDONLY | os.O_DIRECT)
    try:
        for nr in readers:
            req, done = aligned(2 + ring * slot_words), aligned(512)
            pinned = (ctypes.c_void_p * n)(*(store.pinned[k].data_ptr() for k in names))
            pitch = (ctypes.c_long * n)(*(store.pitch[k] for k in names))
            h = lib.ssd_start(fd, ctypes.c_void_p(req.ctypes.data), ctypes.c_void_p(done.ctypes.data), ring, block,
                              store.num_layers, store.num_experts, store.rows, rb, n, pinned, pitch, nr - 1)
            if not h:
                out["readers"][str(nr)] = "ssd_start failed"
                continue
            seq = 0

            def publish(k, first_row):
                nonlocal seq
                seq += 1
                rec = rng.choice(records, size=k, replace=False)
                base = 2 + (seq % ring) * slot_words
                req[base + 2 : base + 2 + block] = -1
                req[base + 2 : base + 2 + k] = rec % store.num_experts  # layer taken from the first
                req[base + 1] = int(rec[0] // store.num_experts)
                req[base + 2 + block : base + 2 + block + k] = first_row + np.arange(k)
                req[base] = seq
                return seq

            def wait(s_):
                t_end = time.perf_counter() + 30.0
                while int(done[0]) < s_:
                    if time.perf_counter() > t_end:
                        raise RuntimeError(f"server sweep: done stuck at {int(done[0])} < {s_}")

            try:
                wb = store.working_base
                # 8-record requests, two outstanding
                t0 = time.perf_counter()
                pending = [publish(8, wb)]
                reqs = 0
                while time.perf_counter() - t0 < seconds or reqs < 4:
                    pending.append(publish(8, wb + 8 * (len(pending) % 2)))
                    wait(pending.pop(0))
                    reqs += 1
                wait(pending.pop(0))
                reqs += 1
                t8 = time.perf_counter() - t0
                # one record at a time
                t0 = time.perf_counter()
                ones = 0
                while time.perf_counter() - t0 < seconds / 2 or ones < 8:
                    wait(publish(1, wb))
                    ones += 1
                t1 = time.perf_counter() - t0
                b, q, r, c = (ctypes.c_double() for _ in range(4))
                preads, nrd, bounce = ctypes.c_long(), ctypes.c_int(), ctypes.c_int()
                lib.xp_ssd_phase_stats(ctypes.c_void_p(h), ctypes.byref(b), ctypes.byref(q), ctypes.byref(r),
                                       ctypes.byref(c), ctypes.byref(preads), ctypes.byref(nrd), ctypes.byref(bounce))
                err = lib.ssd_error(ctypes.c_void_p(h))
            finally:
                lib.ssd_stop(ctypes.c_void_p(h))
            out["readers"][str(nr)] = {
                "gbps_8_record_requests": round(reqs * 8 * rb / t8 / 1e9, 3),
                "ms_per_1_record_request": round(t1 / ones * 1e3, 3),
                "read_s": round(r.value, 3), "copy_s": round(c.value, 3), "queue_s": round(q.value, 3),
                "preads": preads.value, "bounce": bool(bounce.value),
                "error": err.decode() if err else None,
            }
    finally:
        os.close(fd)
    log(f"server sweep: {out}")
    return out


def _o_direct_ok(d: str) -> bool:
    """Whether files in directory d can be read with O_DIRECT (a 4 KiB probe file)."""
    probe = os.path.join(d, f"xp_odirect_{os.getpid()}.bin")
    try:
        with open(probe, "wb") as f:
            f.write(b"\0" * 4096)
        fd = os.open(probe, os.O_RDONLY | os.O_DIRECT)
        try:
            buf = mmap.mmap(-1, 4096)
            os.readv(fd, [buf])
        finally:
            os.close(fd)
        return True
    except OSError:
        return False
    finally:
        if os.path.exists(probe):
            os.unlink(probe)


def paging_dir(args) -> tuple[str | None, str]:
    """The directory for the paging file: --paging-dir when given, else the one of $TMPDIR,
    /tmp, /var/tmp and the repository with the most free space that takes O_DIRECT reads.
    Returns (directory or None, what was considered)."""
    if args.paging_dir:
        return args.paging_dir, f"--paging-dir {args.paging_dir}"
    seen, best, notes = set(), None, []
    for d in (os.environ.get("TMPDIR"), "/tmp", "/var/tmp", ROOT):
        if not d or not os.path.isdir(d):
            continue
        real = os.path.realpath(d)
        if real in seen:
            continue
        seen.add(real)
        try:
            free = shutil.disk_usage(d).free
        except OSError:
            continue
        ok = _o_direct_ok(d)
        notes.append(f"{d}: {free / 2**30:.1f} GiB free{'' if ok else ', no O_DIRECT'}")
        if ok and (best is None or free > best[1]):
            best = (d, free)
    return (best[0] if best else None), "; ".join(notes)


def bench_tiered(args, dev, decode_steps: int | None = None):
    """The compressed tier: 40 layers x 256 experts, 32 cache slots, 128 RAM slots holding rows
    compressed at pitch 0.89, the rest in a paging file read with O_DIRECT by the host server.

    The disk's ceiling for record reads is measured first on the same file. Prefill: one
    2048-token prompt (hidden states bf16 N(0,1), top-8 of random logits, softmax weights), every
    layer through the 64-row working slab in chunks; each layer's output is checked bit for bit
    against a one-shot run over all its experts. Then the decode trace."""
    from vllm_expert_pager import moe
    from vllm_expert_pager import pager as pg

    c = QWEN
    L, E, H, k = c["layers"], c["experts"], c["hidden"], c["topk"]
    T = args.prefill_tokens
    need = L * E * (1_867_776 + 933_888)  # records at pitch 0.89
    pdir, considered = paging_dir(args)
    if pdir is None:
        return {"skipped": f"no directory for the paging file takes O_DIRECT reads ({considered})"}
    try:
        free = shutil.disk_usage(pdir).free
    except OSError as e:
        return {"skipped": f"paging directory {pdir}: {e}"}
    if free < need + (4 << 30):
        return {"skipped": f"the paging file needs {need / 2**30:.1f} GiB and the roomiest directory has "
                           f"{free / 2**30:.1f} GiB free (4 GiB kept spare; {considered})"}
    log(f"paging file in {pdir} ({considered})")
    path = os.path.join(pdir, f"xp_paging_{os.getpid()}.bin")
    settings = pg.Settings(cache_slots=32, ram_slots=128, ssd_path=path, compress="on", pitch_ratio=0.89,
                           working_rows=64, log_interval=0)
    pager, layers, weights = build_paged_model(dev, settings, keep_weights=True)
    store = pager.store
    try:
        ceiling = disk_ceiling(path, store.record_bytes, L * E)
        loaded = disk_ceiling_loaded(path, store.record_bytes, L * E, dev)
        sweep = server_sweep(store, path)
        g = torch.Generator(device=dev).manual_seed(77)
        xs, ws, ids = [], [], []
        for l in range(L):
            xs.append(torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16))
            top, i = torch.randn((T, E), generator=g, device=dev).topk(k, dim=1)
            ws.append(torch.softmax(top, dim=1).float().contiguous())
            ids.append(i)
        torch.cuda.synchronize()
        f0, r0, io0 = store.fetches, store.reads, store.io_seconds
        ph0 = store.phase_stats()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        outs = [layers[l].forward(xs[l], ws[l], ids[l]) for l in range(L)]
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = e0.elapsed_time(e1)
        exact = sum(
            bool(torch.equal(outs[l].view(torch.int16), moe.fused_moe(xs[l], ws[l], ids[l], *weights[l]).view(torch.int16)))
            for l in range(L)
        )
        prefill = {
            "workload": f"40-layer prefill of one {T}-token prompt (bf16 N(0,1) hidden states, top-8 of 256 "
                        "experts, softmax weights), 32 cache slots, 64 working rows, 128 compressed RAM slots, "
                        "the other experts read from the paging file",
            "ms": round(ms, 2),
            "wall_s": round(wall, 3),
            "ms_per_layer": round(ms / L, 3),
            "tokens_per_s": round(T / (ms * 1e-3), 1),
            "ssd_fetches": store.fetches - f0,
            "ssd_reads": store.reads - r0,
            "ssd_io_seconds": round(store.io_seconds - io0, 3),
            "ssd_phases": _phase_delta(store.phase_stats(), ph0),
            "layers_bit_exact_vs_one_shot": f"{exact}/{L}",
        }
        log(f"prefill: {prefill}")
        if exact != L:
            raise SystemExit("chunked prefill differs from the one-shot run")
        del xs, ws, ids, outs, weights
        steps = decode_steps or args.decode_steps
        decode = decode_trace(args, dev, pager, layers,
                              "40-layer decode trace, 256 experts x 3 MiB, 32 cache slots, 128 RAM slots of "
                              "rows compressed at pitch 0.89, the rest read from the paging file (O_DIRECT), "
                              f"batch 1, top-8, Zipf(1.1) with 0.7 reuse, {steps} steps in one "
                              "captured hipGraph per step", steps=steps, paging_steps=min(steps, 300))
        # The server's read rate while it has a request in flight (records read x record bytes /
        # busy seconds; requests overlap, so the summed request time would undercount), against
        # the disk's ceiling at the server's own depth (its reader threads) and at 1 (a decode
        # step's miss is read alone).
        rb = store.record_bytes
        tops = ceiling.get("threads_gbps", {})
        ltops = loaded.get("threads_gbps", {})
        for tgt, reads, phases in ((prefill, prefill["ssd_reads"], prefill["ssd_phases"]),
                                   (decode, (decode.get("ssd") or {}).get("reads", 0),
                                    (decode.get("ssd") or {}).get("phases", {}))):
            busy = phases.get("busy_s", 0.0)
            rate = reads * rb / busy / 1e9 if busy > 0 else None
            tgt["ssd_gbps_while_reading"] = round(rate, 3) if rate else None
            for name, depth in (("server_depth", str(store.readers)), ("1", "1")):
                for kind, table in (("disk_ceiling", tops), ("loaded_disk_ceiling", ltops)):
                    top = table.get(depth)
                    tgt[f"ssd_frac_of_{kind}_{name}"] = (
                        round(rate / top, 3) if rate and isinstance(top, float) else None)
        server = {"readers": store.readers, "sized_from_probe_gbps": store.reader_probe}
        return {"disk_ceiling": ceiling, "disk_ceiling_under_host_link_load": loaded, "server": server,
                "server_sweep": sweep, "prefill": prefill, "decode": decode}
    finally:
        pager.close()
        if os.path.exists(path):
            os.unlink(path)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--rows", type=int, default=256)
    ap.add_argument("--cpu-rows", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--gather-steps", type=int, default=10)
    ap.add_argument("--moe-steps", type=int, default=5)
    ap.add_argument("--only-decode", action="store_true")
    ap.add_argument("--only-moe", action="store_true")
    ap.add_argument("--only-model", action="store_true")
    ap.add_argument("--only-encode", action="store_true")
    ap.add_argument("--tiered", action="store_true",
                    help="run only the compressed-tier legs (disk ceiling, 2048-token prefill, decode trace; "
                         "needs ~30 GB of disk for the paging file)")
    ap.add_argument("--no-tiered", action="store_true",
                    help="leave the compressed-tier legs out of the default run")
    ap.add_argument("--tiered-decode-steps", type=int, default=2000,
                    help="decode steps of the compressed tier in the default run (the configured 2000)")
    ap.add_argument("--prefill-tokens", type=int, default=2048)
    ap.add_argument("--paging-dir", default=None,
                    help="directory for the tiered leg's paging file (default: the roomiest of $TMPDIR, "
                         "/tmp, /var/tmp and the repository that takes O_DIRECT reads)")
    ap.add_argument("--decode-steps", type=int, default=2000)
    ap.add_argument("--decode-warmup", type=int, default=20)
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="before the legs, copy this many MiB device to device three times "
                         "(the plain copy that scales the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        raise SystemExit(2)
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    from vllm_expert_pager import _native

    _native.lib()  # fails loudly if the HIP library is not built
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cores = len(os.sched_getaffinity(0))

    if args.copy_probe_mib:
        n = args.copy_probe_mib << 20
        a = torch.randint(0, 255, (n,), dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        for _ in range(3):
            torch.bitwise_not(a, out=b)
        torch.cuda.synchronize()
        del a, b
        log(f"copy probe: 3 device copies and 3 elementwise passes of {args.copy_probe_mib} MiB")
    if args.only_moe:
        print(json.dumps({"moe": bench_moe(args, dev)}), flush=True)
        return
    if args.only_model:
        print(json.dumps({"model_decode": bench_model_decode(args, dev)}), flush=True)
        return
    if args.only_encode:
        print(json.dumps({"encode": bench_encode(args, dev, cores)}), flush=True)
        return
    if args.tiered:
        print(json.dumps({"tiered": bench_tiered(args, dev)}), flush=True)
        return
    dec = bench_decode(args, dev, cores)
    extras = {}
    if not args.only_decode:
        extras["encode"] = bench_encode(args, dev, cores)
        extras["gather"] = bench_gather(args, dev)
        extras["acquire"] = bench_acquire(args, dev)
        extras["moe"] = bench_moe(args, dev)
        extras["model_decode"] = bench_model_decode(args, dev)
        try:
            extras["model_decode_compressed"] = bench_model_decode_compressed(args, dev)
        except (RuntimeError, MemoryError, ValueError) as e:  # reported, so the other legs still print
            extras["model_decode_compressed"] = {"failed": f"{type(e).__name__}: {e}"}
            log(f"compressed RAM-tier decode trace failed: {e}")
        if not args.no_tiered:
            extras["tiered"] = bench_tiered(args, dev, args.tiered_decode_steps)
    line = {
        "metric": "Huffman decode GB/s (% HBM peak); gather GB/s; acquire us/layer; decode tok/s",
        "value": round(dec["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic",
        "config": {
            "workload": f"codec only: batched GPU expansion of {args.rows} compressed experts per launch "
                        "(w13 fp8 1024x2048 + w2 fp8 2048x512, N(0,0.02) e4m3 with 128x128 block scales, "
                        "pitch 0.89)",
            "rows_per_launch": args.rows,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(dec["gbps"], 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(dec["gbps"] / HBM_PEAK_GBPS, 4),
            "traffic": decode_traffic(args.rows),
            "valu": decode_valu(args.rows, dec["alg_bytes"], dec["gbps"], dec["n_bytes"]),
        },
        "cpu_baseline": dec["cpu"],
        "decode_warmup": dec["warm"],
        "decode_raw_output_gbps": round(dec["raw_gbps"], 2),
        "decode_gbps_by_rows": dec["sweep"],
        "decode_us_by_rows": dec["sweep_us"],
        "decode_from_ram_us_by_rows": dec["ram_us"],
        **extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
