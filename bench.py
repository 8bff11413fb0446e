#!/usr/bin/env python3
"""Benchmark of the Pet JSON codec on one MI355X.

Headline line (the driver's contract): BASELINE.json configs[2] — the full
nested encode of 10M Pets (category, photoUrls, tags, escapes) from SoA
columns already resident in HBM into one JSON array, records/s; this is the
workload the north-star target names.  The same JSON object also carries the
flat-encode, skewed and NDJSON-decode
figures under "workloads", each with its own fraction of the HBM roofline,
the roofline of the headline kernel measured with HIP events on the codec's
stream, and the CPU restatement timed on this host's cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload nested|flat|decode|skew|options]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "micronaut3-bug_amd"))

METRIC = "records/s and output GB/s (% of HBM peak) for 10M-Pet encode/decode, 1 GPU"
HBM_PEAK_GBPS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def col_bytes(cols):
    return cols.input_bytes()


def run_encode(codec, cols_dev, fmt, steps, warmup):
    import torch
    import petjson as pj
    need = codec.encode_size(cols_dev, fmt)
    out = torch.empty(need + 4, dtype=torch.uint8, device="cuda")
    for _ in range(warmup):
        codec.encode(cols_dev, fmt, out=out)
    torch.cuda.synchronize()
    kern = []
    t0 = time.perf_counter()
    for _ in range(steps):
        codec.encode(cols_dev, fmt, out=out)
        kern.append(codec.timings()[0])      # the whole device pipeline, HIP events on the codec stream
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    return need, wall, sum(kern) / len(kern), out


def encode_workload(codec, config, n, steps, warmup):
    import petjson as pj
    log(f"[bench] generating config {config}, {n} records")
    cols = pj.generate(config, n)
    dev = cols.to_device()
    in_bytes = col_bytes(cols)
    out_bytes, wall, kms, _ = run_encode(codec, dev, pj.FORMAT_ARRAY, steps, warmup)
    alg = in_bytes + out_bytes
    # the host entry point on the same columns (PCIe-inclusive; not the headline)
    hostr = host_encode_rates(codec, cols, in_bytes, out_bytes)
    res = {
        "records": n, "records_per_s": n / wall, "ms_per_step": wall * 1e3,
        "output_bytes": out_bytes, "input_bytes": in_bytes,
        "output_GBps": out_bytes / wall / 1e9, "output_frac_hbm": out_bytes / wall / 1e9 / HBM_PEAK_GBPS,
        "kernel_ms": kms, "kernel_alg_GBps": alg / (kms * 1e-3) / 1e9,
        "kernel_alg_frac_hbm": alg / (kms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
        "host_entry_point": hostr,
    }
    return cols, res


def host_encode_rates(codec, cols, in_bytes, out_bytes, reps=3):
    """pj_encode_host on the host columns into a buffer sized by
    pj_encode_bound: with pageable buffers (copied through the library's
    pinned bounce buffers) and with pinned ones (pj_host_alloc, moved by DMA
    directly), beside a plain pinned D2H copy of the output's size (the
    larger of the two directions).  Inputs over 512 MiB stream in segments,
    so the copies in and out overlap.  Medians of reps."""
    import ctypes as C
    import numpy as np
    import torch
    import petjson as pj
    med = lambda v: sorted(v)[len(v) // 2]
    pin = torch.empty(out_bytes, dtype=torch.uint8, pin_memory=True)
    d = torch.empty(out_bytes, dtype=torch.uint8, device="cuda")
    d2h = []
    for _ in range(reps):
        torch.cuda.synchronize(); t0 = time.perf_counter(); pin.copy_(d, non_blocking=True); torch.cuda.synchronize()
        d2h.append(out_bytes / (time.perf_counter() - t0) / 1e9)
    del pin, d
    torch.cuda.empty_cache()
    s, b = cols.struct(), C.c_uint64(0)
    codec._check(codec.L.pj_encode_bound(C.byref(s), pj.FORMAT_ARRAY, C.byref(b)))
    out = {}
    for kind in ("pageable", "pinned"):
        if kind == "pageable":
            hc, buf = cols, np.ones(b.value, np.uint8)
        else:
            hc = pj.Columns(cols.n_pets, {}, dict(cols.caps))
            for k, v in cols.arrays.items():
                if v is not None:
                    a = pj.host_array(len(v), v.dtype)
                    a[:] = v
                    v = a
                hc.arrays[k] = v
            buf = pj.host_array(b.value, np.uint8)
            buf[:] = 1
        st, n = hc.struct(), C.c_uint64(0)
        ms, ok = [], True
        for _ in range(reps + 1):
            t0 = time.perf_counter()
            rc = codec.L.pj_encode_host(codec.ctx, C.byref(st), pj.FORMAT_ARRAY, C.c_void_p(buf.ctypes.data), buf.size,
                                        C.byref(n))
            ms.append((time.perf_counter() - t0) * 1e3)
            ok = ok and rc == 0 and n.value == out_bytes
        m = med(ms[1:])
        out["encode_host_" + kind] = {"ms": m, "moved_GBps": (in_bytes + out_bytes) / m / 1e6, "ok": bool(ok)}
        del hc, buf
    out["pinned_d2h_copy_GBps"] = med(d2h)
    out["pinned_d2h_copy_of_output_ms"] = out_bytes / med(d2h) / 1e6
    out["pinned_encode_frac_of_d2h_copy"] = out["pinned_d2h_copy_of_output_ms"] / out["encode_host_pinned"]["ms"]
    return out


def decode_workload(codec, n, steps, warmup):
    """NDJSON from the nested generator, 0.1% of lines corrupted."""
    import numpy as np
    import torch
    import petjson as pj
    log(f"[bench] generating config 4, {n} records")
    cols = pj.generate(4, n)
    dev = cols.to_device()
    text = codec.encode(dev, pj.FORMAT_NDJSON)
    host = text.cpu().numpy().copy()
    del dev, text
    torch.cuda.empty_cache()
    lines, codes = pj.corrupt_ndjson(host, 0xBAD, 0.001)
    data = torch.from_numpy(host).cuda()
    host_text = host.tobytes()
    del host
    sz = cols.sizes()
    caps = {"cap_pets": n, "cap_name_bytes": sz["name_bytes"], "cap_cat_name_bytes": sz["cat_name_bytes"],
            "cap_urls": sz["n_urls"], "cap_url_bytes": sz["url_bytes"], "cap_tags": sz["n_tags"],
            "cap_tag_name_bytes": sz["tag_name_bytes"]}
    bufs = codec.decode_buffers(caps, max(16, 2 * len(lines)))
    for _ in range(warmup):
        codec.decode(data, out=bufs)
    torch.cuda.synchronize()
    names = ["k_dec_lines", "k_dec_block", "k_dec_bscan", "k_dec_write", "k_dec_long", "k_dec_errcode"]
    per = {k: [] for k in names}
    t0 = time.perf_counter()
    for _ in range(steps):
        dcols, el, ec, res = codec.decode(data, out=bufs)
        # [total, fill, k_dec_lines, host gap, fill, k_dec_block, k_dec_bscan, k_dec_write, k_dec_long,
        #  k_dec_errcode] (HIP events on the codec stream)
        tm = codec.timings()
        for k, i in zip(names, (2, 5, 6, 7, 8, 9)):
            per[k].append(tm[i])
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    ok = (res.n_errors == len(lines) and np.array_equal(el.cpu().numpy().astype(np.uint64), lines)
          and np.array_equal(ec.cpu().numpy(), codes) and res.n_pets == n - len(lines))
    out_bytes = sum(int(dcols[k].numel()) * dcols[k].element_size() for k in pj.COLS)
    in_bytes = int(data.numel())
    kern = {k + "_ms": sum(v) / len(v) for k, v in per.items()}
    ksum = sum(kern.values())
    kern["kernels_sum_ms"] = ksum
    kern["k_dec_lines_GBps"] = in_bytes / (kern["k_dec_lines_ms"] * 1e-3) / 1e9
    kern["alg_frac_hbm_kernels"] = (in_bytes + out_bytes) / (ksum * 1e-3) / 1e9 / HBM_PEAK_GBPS
    # the host entry point on the same text (PCIe-inclusive; not the headline)
    del bufs
    torch.cuda.empty_cache()
    hostr = host_decode_rates(codec, np.frombuffer(host_text, np.uint8), caps, max(16, 2 * len(lines)), int(res.n_pets))
    del data
    torch.cuda.empty_cache()
    arr = array_decode_rates(codec, cols, caps, steps, warmup)
    r = {"records": int(res.n_lines), "records_per_s": res.n_lines / wall, "ms_per_step": wall * 1e3,
         "input_bytes": in_bytes, "output_bytes": out_bytes, "input_GBps": in_bytes / wall / 1e9,
         "alg_GBps": (in_bytes + out_bytes) / wall / 1e9,
         "alg_frac_hbm": (in_bytes + out_bytes) / wall / 1e9 / HBM_PEAK_GBPS,
         "invalid_records": int(res.n_errors), "errors_match_generator": bool(ok),
         "lines_general_parser": int(res.n_general), "kernels": kern,
         "host_entry_point": hostr, "array_document": arr}
    return r


def array_decode_rates(codec, cols, caps, steps, warmup):
    """The same records as one JSON array document (readValue(bytes,
    List<Pet>)): the frame kernels cut it into elements, then the line
    stages decode them.  Columns compared with the generator's."""
    import numpy as np
    import torch
    import petjson as pj
    dev = cols.to_device()
    doc = codec.encode(dev, pj.FORMAT_ARRAY)
    del dev
    torch.cuda.empty_cache()
    bufs = codec.decode_buffers(caps, 16)
    for _ in range(warmup):
        codec.decode_array(doc, out=bufs)
    torch.cuda.synchronize()
    kms = []
    t0 = time.perf_counter()
    for _ in range(steps):
        dcols, el, ec, res = codec.decode_array(doc, out=bufs)
        kms.append(codec.timings()[0])                 # the whole pipeline, HIP events on the codec stream
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    h = dcols.to_host()
    same = res.n_errors == 0 and all(np.array_equal(h[k], cols[k]) for k in pj.COLS if cols[k] is not None)
    in_bytes = int(doc.numel())
    out_bytes = sum(int(dcols[k].numel()) * dcols[k].element_size() for k in pj.COLS)
    k = sum(kms) / len(kms)
    r = {"records": int(res.n_pets), "input_bytes": in_bytes, "output_bytes": out_bytes, "ms_per_step": wall * 1e3,
         "pipeline_ms": k, "alg_frac_hbm": (in_bytes + out_bytes) / (k * 1e-3) / 1e9 / HBM_PEAK_GBPS,
         "roundtrip_bit_exact": bool(same)}
    del doc, bufs, dcols
    torch.cuda.empty_cache()
    return r


def host_decode_rates(codec, text, caps, err_cap, n_pets, reps=3):
    """pj_decode_host on host input, outputs preallocated (and touched): with
    pageable buffers (copied through the library's pinned bounce buffers)
    and with pinned ones (pj_host_alloc, moved by DMA directly), beside
    plain pinned H2D / D2H copies of the input's size.  Medians of reps."""
    import ctypes as C
    import numpy as np
    import torch
    import petjson as pj
    N = int(text.size)
    med = lambda v: sorted(v)[len(v) // 2]
    pin = torch.empty(N, dtype=torch.uint8, pin_memory=True)
    d = torch.empty(N, dtype=torch.uint8, device="cuda")
    h2d, d2h = [], []
    for _ in range(reps):
        torch.cuda.synchronize(); t0 = time.perf_counter(); d.copy_(pin, non_blocking=True); torch.cuda.synchronize()
        h2d.append(N / (time.perf_counter() - t0) / 1e9)
        t0 = time.perf_counter(); pin.copy_(d, non_blocking=True); torch.cuda.synchronize()
        d2h.append(N / (time.perf_counter() - t0) / 1e9)
    del pin, d
    torch.cuda.empty_cache()
    cp, cu, ct = caps["cap_pets"], caps["cap_urls"], caps["cap_tags"]
    sizes = {"id": cp, "flags": cp, "status": cp, "name_off": cp + 1, "name_bytes": caps["cap_name_bytes"],
             "cat_id": cp, "cat_flags": cp, "cat_name_off": cp + 1, "cat_name_bytes": caps["cap_cat_name_bytes"],
             "photo_off": cp + 1, "url_off": cu + 1, "url_bytes": caps["cap_url_bytes"], "tag_off": cp + 1,
             "tag_id": ct, "tag_flags": ct, "tag_name_off": ct + 1, "tag_name_bytes": caps["cap_tag_name_bytes"]}
    out = {}
    for kind in ("pageable", "pinned"):
        alloc = (lambda n, t: np.ones(max(1, n), t)) if kind == "pageable" else pj.host_array
        inp = text if kind == "pageable" else alloc(N, np.uint8)
        if kind == "pinned":
            inp[:] = text
        cols = pj.Columns(0, {k: alloc(v, pj.DTYPES[k]) for k, v in sizes.items()}, dict(caps))
        for a in cols.arrays.values():
            a[:] = 1
        el, ec = alloc(err_cap, np.uint64), alloc(err_cap, np.uint8)
        ms, ok = [], True
        for _ in range(reps + 1):
            st = cols.struct()
            res = pj.DecodeResult()
            t0 = time.perf_counter()
            rc = codec.L.pj_decode_host(codec.ctx, C.c_void_p(inp.ctypes.data), N, C.byref(st),
                                        C.c_void_p(el.ctypes.data), C.c_void_p(ec.ctypes.data), err_cap, C.byref(res))
            ms.append((time.perf_counter() - t0) * 1e3)
            ok = ok and rc == 0 and res.n_pets == n_pets
        m = med(ms[1:])
        out["decode_host_" + kind] = {"ms": m, "input_GBps": N / m / 1e6, "ok": bool(ok)}
        del cols, inp, el, ec
    out["pinned_h2d_copy_GBps"] = med(h2d)
    out["pinned_d2h_copy_GBps"] = med(d2h)
    out["pinned_decode_frac_of_h2d_copy"] = out["decode_host_pinned"]["input_GBps"] / out["pinned_h2d_copy_GBps"]
    out["pageable_decode_frac_of_h2d_copy"] = out["decode_host_pageable"]["input_GBps"] / out["pinned_h2d_copy_GBps"]
    return out


def _timed(fn, budget_s, threads):
    """Run fn repeatedly on `threads` host threads for about budget_s seconds
    (the oracle's ctypes calls release the GIL); returns (calls, seconds)."""
    import threading
    fn()                            # warm: library load, first-touch allocations
    counts = [0] * threads
    t0 = time.perf_counter()

    def work(k):
        while time.perf_counter() - t0 < budget_s:
            fn()
            counts[k] += 1

    ts = [threading.Thread(target=work, args=(k,)) for k in range(threads)]
    for th in ts:
        th.start()
    for th in ts:
        th.join()
    return sum(counts), time.perf_counter() - t0


def host_cores():
    """Threads for the all-core CPU leg: the CPUs this process may run on,
    bounded by the cgroup CPU quota when one is set (the GPU box grants a
    share of its host; os.cpu_count() shows the whole machine)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    src = "affinity"
    try:
        q, per = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            quota = max(1, int(int(q) // int(per)))
            if quota < n:
                n, src = quota, "cgroup cpu.max quota"
    except (OSError, ValueError):
        pass
    return max(1, n), src


def cpu_model():
    try:
        for l in open("/proc/cpuinfo"):
            if l.startswith("model name"):
                return l.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_rate(fn, units, runs, per_run_s, threads):
    """Median over `runs` timed windows of units/s, fn run on `threads`
    host threads; returns (median rate, all rates)."""
    rates = []
    for _ in range(runs):
        k, e = _timed(fn, per_run_s, threads)
        rates.append(units * k / e)
    rates.sort()
    return rates[len(rates) // 2], rates


def skew_workload(codec, n, steps, warmup, with_decode):
    """2M records with log-normal names (1% of 8-16 KiB names and
    200 tags, 30% escape-heavy UTF-8): NDJSON encode, and with with_decode the
    round trip back to columns, checked bit-exact."""
    import numpy as np
    import torch
    import petjson as pj
    log(f"[bench] generating config 5, {n} records")
    cols = pj.generate(5, n)
    dev = cols.to_device()
    in_bytes = col_bytes(cols)
    out_bytes, wall, kms, out = run_encode(codec, dev, pj.FORMAT_NDJSON, steps, warmup)
    r = {"records": n, "records_per_s": n / wall, "ms_per_step": wall * 1e3, "input_bytes": in_bytes,
         "output_bytes": out_bytes, "kernel_ms": kms,
         "kernel_alg_GBps": (in_bytes + out_bytes) / (kms * 1e-3) / 1e9,
         "kernel_alg_frac_hbm": (in_bytes + out_bytes) / (kms * 1e-3) / 1e9 / HBM_PEAK_GBPS}
    if with_decode:
        text = out[:out_bytes]
        res = None
        # outputs allocated once and one untimed call first, as for configs[3]
        sz = cols.sizes()
        caps = {"cap_pets": n, "cap_name_bytes": sz["name_bytes"], "cap_cat_name_bytes": sz["cat_name_bytes"],
                "cap_urls": sz["n_urls"], "cap_url_bytes": sz["url_bytes"], "cap_tags": sz["n_tags"],
                "cap_tag_name_bytes": sz["tag_name_bytes"]}
        bufs = codec.decode_buffers(caps, 4096)
        codec.decode(text, out=bufs)
        torch.cuda.synchronize()
        dsteps = max(1, steps // 2)
        dev_ms = []
        t0 = time.perf_counter()
        for _ in range(dsteps):
            dcols, el, ec, res = codec.decode(text, out=bufs)
            dev_ms.append(codec.timings()[0])    # first to last HIP event of the call
        torch.cuda.synchronize()
        dwall = (time.perf_counter() - t0) / dsteps
        h = dcols.to_host()
        same = res.n_errors == 0 and all(np.array_equal(h[k], cols[k]) for k in pj.COLS if cols[k] is not None)
        dkms = sum(dev_ms) / len(dev_ms)
        r.update({"decode_ms_per_step": dwall * 1e3, "decode_device_ms": dkms, "roundtrip_bit_exact": bool(same),
                  "decode_alg_GBps": (out_bytes + in_bytes) / dwall / 1e9,
                  "decode_device_alg_frac_hbm": (out_bytes + in_bytes) / (dkms * 1e-3) / 1e9 / HBM_PEAK_GBPS})
        # the same lines with 0.1% corrupted: the invalid lines' first-error
        # codes (k_dec_errcode, the last kernel of the call) against the
        # generator's list of what it corrupted
        host = text.cpu().numpy().copy()
        lines, codes = pj.corrupt_ndjson(host, 0x5EED5, 0.001)
        bad = torch.from_numpy(host).cuda()
        del host
        dms, ems = [], []
        for _ in range(max(2, steps // 2)):
            dcols, el, ec, res = codec.decode(bad, err_cap=2 * len(lines))
            tm = codec.timings()
            dms.append(tm[0])
            ems.append(tm[-1])
        ok = (res.n_errors == len(lines) and np.array_equal(el.cpu().numpy().astype(np.uint64), lines) and
              np.array_equal(ec.cpu().numpy(), codes))
        r["corrupted_decode"] = {"invalid_lines": int(len(lines)), "errors_match_generator": bool(ok),
                                 "decode_pipeline_ms": sum(dms[1:]) / len(dms[1:]),
                                 "k_dec_errcode_ms": sum(ems[1:]) / len(ems[1:])}
        del bad
    del dev, out
    torch.cuda.empty_cache()
    return r


def _cpu_leg(fn, units, budget_s):
    cores, src = host_cores()
    per = budget_s / 10.0                     # 5 windows on 1 thread + 5 on every core
    m1, r1 = _median_rate(fn, units, 5, per, 1)
    mn, rn = _median_rate(fn, units, 5, per, cores)
    return m1, r1, mn, rn, cores, src


def cpu_baseline_encode(config, n_sample, budget_s=10.0):
    """Oracle (C restatement) encode of a bounded sample of the same
    configuration: median of 5 timed windows on one thread, then on every
    core this process is granted (one sample per thread)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_py as orc
    import petjson as pj
    sample = pj.generate(config, n_sample)
    fn = lambda: orc.encode(sample, pj.FORMAT_ARRAY)
    m1, r1, mn, rn, cores, src = _cpu_leg(fn, n_sample, budget_s)
    return {"value": mn, "unit": "records/s", "cores": cores, "kind": "port",
            "single_thread_value": m1, "cpu_model": cpu_model(), "nproc": os.cpu_count(),
            "cores_source": src, "runs_1_thread": r1, "runs_all_cores": rn,
            "sample": f"{n_sample} records of configs[{config - 1}], encoded by oracle/pj_oracle.c (C restatement "
                      f"of the serde/Jackson rules; the reference is Java and no JVM is available); median of 5 "
                      f"windows of {budget_s / 10:.1f}s on 1 thread and on {cores} threads"}


def _model_bytes(cols):
    """Bytes of an Order / User column set (host numpy)."""
    tot = cols.present.nbytes if cols.present is not None else 0
    for c in cols.col:
        tot += c.nbytes
    for b in cols.bytes:
        tot += b.nbytes if b is not None else 0
    return tot


def _kernel_ms(codec, fn, steps, warmup, idx):
    """Mean of one HIP-event interval (idx into Codec.timings()) over steps calls."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ms = []
    for _ in range(steps):
        r = fn()
        ms.append(codec.timings()[idx])
    return sum(ms) / len(ms), r


def option_workloads(codec, steps):
    """The non-headline paths at a real size, each with its kernel time and
    algorithmic bytes (columns in + JSON out): pretty printing and the
    findPetsByStatus body over configs[2] records, and the Order / User
    models' encode and decode (4M records each, seeded)."""
    import torch
    import petjson as pj
    res = {}
    cols = pj.generate(3, 10_000_000)
    dev = cols.to_device()
    in_bytes = col_bytes(cols)
    ms, out = _kernel_ms(codec, lambda: codec.encode(dev, pj.FORMAT_PRETTY), steps, 1, -1)
    alg = in_bytes + out.numel()
    res["pretty_encode"] = {"records": cols.n_pets, "kernel": "k_encode_rows<PRETTY>", "kernel_ms": ms,
                            "output_bytes": out.numel(), "alg_frac_hbm": alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS}
    del out
    ms_sel, (body, m) = _kernel_ms(codec, lambda: codec.encode_by_status(dev, 1, pj.FORMAT_ARRAY), steps, 1, -1)
    sel_ms = codec.timings()[-2]                   # k_select_status, same call
    res["by_status_encode"] = {"records": cols.n_pets, "selected": m, "status_mask": 1,
                               "kernel": "k_select_status + k_encode_rows", "select_ms": sel_ms, "encode_ms": ms_sel,
                               "output_bytes": body.numel()}
    del body, dev, cols
    torch.cuda.empty_cache()
    # every property present and empty strings kept (ALWAYS), so that the
    # decoded columns must equal the encoded ones exactly
    codec.set_options(pj.INCLUDE_ALWAYS)
    for name, model in (("order", pj.MODEL_ORDER), ("user", pj.MODEL_USER)):
        mc = pj.generate_model(model, 4_000_000, seed=1, null_rate=0.0, fancy=False)
        md = mc.to_device()
        ib = _model_bytes(mc)
        ems, text = _kernel_ms(codec, lambda: codec.encode_model(md, pj.FORMAT_NDJSON), steps, 1, -1)
        text = text.clone()
        dms, (dc, el, ec, r) = _kernel_ms(codec, lambda: codec.decode_model(model, text), steps, 1, -1)
        n = mc.n
        same = r.n_pets == n and r.n_errors == 0 and torch.equal(dc.present[:n], md.present[:n])
        for k, (_, kind) in enumerate(mc.props):
            cnt = n + 1 if kind == "str" else n
            same = same and torch.equal(dc.col[k][:cnt], md.col[k][:cnt])
            if kind == "str":
                nb = int(mc.col[k][-1])
                same = same and torch.equal(dc.bytes[k][:nb], md.bytes[k][:nb])
        res[name + "_encode"] = {"records": mc.n, "kernel": "k_encode_model", "kernel_ms": ems,
                                 "output_bytes": text.numel(),
                                 "alg_frac_hbm": (ib + text.numel()) / (ems * 1e-3) / 1e9 / HBM_PEAK_GBPS}
        res[name + "_decode"] = {"records": mc.n, "kernel": "k_mdec_count + k_mdec_scan + k_mdec_write",
                                 "kernels_ms": dms, "roundtrip_columns_equal": bool(same),
                                 "alg_frac_hbm": (ib + text.numel()) / (dms * 1e-3) / 1e9 / HBM_PEAK_GBPS}
        del md, text, dc
        torch.cuda.empty_cache()
    codec.set_options()
    return res


def cpu_baseline_decode(n_sample, budget_s=10.0):
    """Oracle decode of a bounded sample of the decode workload (config 4
    generator, NDJSON, 0.1% corrupted): median of 5 windows on one thread,
    then on every granted core."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import numpy as np
    import oracle_py as orc
    import petjson as pj
    cols = pj.generate(4, n_sample)
    text = np.frombuffer(orc.encode(cols, pj.FORMAT_NDJSON), dtype=np.uint8).copy()
    pj.corrupt_ndjson(text, 0xBAD, 0.001)
    data = text.tobytes()
    fn = lambda: orc.decode(data)
    m1, r1, mn, rn, cores, src = _cpu_leg(fn, n_sample, budget_s)
    return {"value": mn, "unit": "records/s", "cores": cores, "kind": "port",
            "single_thread_value": m1, "cpu_model": cpu_model(), "nproc": os.cpu_count(),
            "cores_source": src, "runs_1_thread": r1, "runs_all_cores": rn,
            "input_GBps_all_cores": mn * len(data) / n_sample / 1e9,
            "sample": f"{n_sample} NDJSON lines ({len(data)} bytes) of the decode workload, decoded by "
                      f"oracle/pj_oracle.c; median of 5 windows of {budget_s / 10:.1f}s on 1 thread and on "
                      f"{cores} threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="nested", choices=["flat", "nested", "decode", "skew", "options"],
                    help="headline workload; 'decode' runs only the NDJSON decode and 'skew' only the "
                         "configs[4] encode + decode round trip, 'options' only the pretty, findPetsByStatus and "
                         "Order / User paths (for profiling)")
    ap.add_argument("--records", type=int, default=10_000_000)
    ap.add_argument("--decode-records", type=int, default=14_600_000)
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary workloads")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode workloads")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="only run a plain device-to-device copy of BYTES (4x), to scale rocprof "
                         "FETCH_SIZE / WRITE_SIZE readings")
    a = ap.parse_args()
    if a.calibrate_copy:
        import torch
        src = torch.ones(a.calibrate_copy, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": a.calibrate_copy}))
        return
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {a.gpus}): the codec runs on one GPU's share "
              f"(records split by row ranges, NDJSON at newlines) and no multi-GPU figure is produced.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import petjson as pj
    codec = pj.Codec(0)
    if a.workload == "skew":
        print(json.dumps({"skew_encode": skew_workload(codec, 2_000_000, a.steps, a.warmup, not a.no_decode)}),
              flush=True)
        codec.close()
        return
    if a.workload == "options":
        print(json.dumps({"options": option_workloads(codec, a.steps)}), flush=True)
        codec.close()
        return
    if a.workload == "decode":
        print(json.dumps({"ndjson_decode": decode_workload(codec, a.decode_records, a.steps, a.warmup),
                          "cpu_baseline_decode": cpu_baseline_decode(50_000, a.cpu_budget)}), flush=True)
        codec.close()
        return
    cfg = 2 if a.workload == "flat" else 3
    cols, head = encode_workload(codec, cfg, a.records, a.steps, a.warmup)
    workloads = {a.workload + "_encode": head}
    if not a.no_extra:
        other = 3 if cfg == 2 else 2
        _, r = encode_workload(codec, other, a.records, max(3, a.steps // 2), 1)
        workloads[("nested" if other == 3 else "flat") + "_encode"] = r
    del cols
    torch.cuda.empty_cache()
    if not a.no_extra:
        workloads["skew_encode"] = skew_workload(codec, 2_000_000, max(3, a.steps // 2), 1, not a.no_decode)
        torch.cuda.empty_cache()
    if not a.no_extra and not a.no_decode:
        workloads["ndjson_decode"] = decode_workload(codec, a.decode_records, max(3, a.steps // 2), 1)
        torch.cuda.empty_cache()
    if not a.no_extra:
        workloads["options"] = option_workloads(codec, max(3, a.steps // 4))
        torch.cuda.empty_cache()
    cpu = cpu_baseline_encode(cfg, 200_000 if cfg == 2 else 50_000, a.cpu_budget)
    cpu_dec = cpu_baseline_decode(50_000, a.cpu_budget) if not a.no_extra else None
    alg = head["input_bytes"] + head["output_bytes"]
    achieved = alg / (head["kernel_ms"] * 1e-3) / 1e9
    traffic = None
    tf = os.path.join(ROOT, "profiles", "k_encode_traffic.json")
    if os.path.exists(tf) and a.records == 10_000_000:
        traffic = json.load(open(tf)).get(a.workload + "_encode", {}).get("traffic")
    traffic_src = ("profiles/k_encode_traffic.json: rocprofv3 FETCH_SIZE + WRITE_SIZE of k_encode on this "
                   "workload, scaled by a plain-copy calibration") if traffic is not None else None
    line = {
        "metric": METRIC,
        "value": head["records_per_s"],
        "unit": "records/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic (seeded generator, BASELINE.json configs)",
        "config": {"workload": ("configs[1] flat encode" if cfg == 2 else "configs[2] nested encode") +
                               f", {a.records} Pets, SoA columns in HBM -> JSON array",
                   "records": a.records, "format": "array"},
        "output_GBps": head["output_GBps"],
        "output_frac_hbm": head["output_frac_hbm"],
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic, "traffic_source": traffic_src,
                     "kernel": "k_encode", "kernel_ms": head["kernel_ms"],
                     "alg_bytes_per_launch": alg},
        "cpu_baseline": cpu,
        "cpu_baseline_decode": cpu_dec,
        "workloads": workloads,
    }
    print(json.dumps(line), flush=True)
    codec.close()


if __name__ == "__main__":
    main()
