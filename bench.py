"""Benchmark of the attention / Gated-DeltaNet hot path on one MI355X.

Headline (BASELINE.json metric "decode attn us/layer + HBM GB/s @ctx 8192; prefill attn TFLOP/s
@8192 tok"): one step = one decode attention layer (config 2: batch 1, 16 q / 2 KV heads,
head_dim 256, f16 KV cache of 8192 positions, seed 1) through it_attn_f16. `value` is its HBM
throughput in algorithmic bytes (K+V f16 + q/gate + out) per second. Beside it the run measures
MTP verify (nt=4), decode at ctx 512, chunked / whole-prompt causal prefill TFLOP/s (config 3) and
the GDN decode step (config 4), and times the CPU restatement of src/cpu.rs on host cores.

Method: every timed sequence is captured once into a HIP graph (torch.cuda.graph) and replayed,
so the figures are device time for back-to-back launches, not Python call overhead; HIP events on
the capture stream bracket the replay. Decode KV caches rotate through 40 distinct copies
(640 MiB) so the 256 MB MALL cannot serve them; GDN states rotate through 160 copies (320 MiB).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
COPY_KIB = 262144   # the calibration copy: 256 MiB read and written
F16_MFMA_PEAK_TFLOPS = 2500.0
NH, NKV, HD = 16, 2, 256
KVD = NKV * HD


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_bytes(n_keys: int, nt: int = 1) -> int:
    """Algorithmic HBM bytes of one decode/verify attention layer: K+V f16 rows once, q+gate f32 in,
    out f32 written."""
    return 2 * n_keys * KVD * 2 + nt * NH * 2 * HD * 4 + nt * NH * HD * 4


def prefill_flops(pos0: int, nt: int) -> int:
    """4*hd*nh*sum_t (pos0+t+1): QK^T and PV over visible keys, masked work not counted."""
    return 4 * HD * NH * sum(pos0 + t + 1 for t in range(nt))


def prep_bytes(nt: int) -> int:
    """Algorithmic HBM bytes of the attention pre-pass: q read and rewritten (f32, query halves only),
    k and v read (f32), K and V rows written (f16)."""
    return nt * (NH * HD * 4 * 2 + 2 * KVD * 4 + 2 * KVD * 2)


def graph_time_ms(torch, fn, reps: int, warm: int = 3) -> float:
    """Capture `fn` (which enqueues work on the current stream) into a graph, replay `warm` times,
    then time one more replay with events on the capture stream. Returns ms per replay."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()   # eager warm-up on the side stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        fn()
    for _ in range(warm):
        g.replay()
    torch.cuda.synchronize()
    best = None
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(s):
            e0.record(s)
            g.replay()
            e1.record(s)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
        best = ms if best is None else min(best, ms)
    return best


def pmc_median(counter: str, bench_args: list, kernel: str, grid: str):
    """Run bench.py once more, as a child process under `rocprofv3 --pmc <counter>` (counters cannot
    be collected in the timed process), and return (median of the counter over the dispatches of
    `kernel` at total grid size `grid`, None) or (None, reason)."""
    import csv, glob, shutil, signal, statistics, subprocess, tempfile
    prof = shutil.which("rocprofv3")
    if not prof:
        return None, "rocprofv3 not found"
    with tempfile.TemporaryDirectory(dir="/tmp") as d:
        cmd = [prof, "--pmc", counter, "-d", d, "-o", "run", "--output-format", "csv", "--", sys.executable,
               os.path.join(ROOT, "bench.py"), "--no-pmc"] + bench_args
        proc = subprocess.Popen(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"), stdout=subprocess.DEVNULL,
                                stderr=subprocess.DEVNULL, start_new_session=True)
        try:
            rc = proc.wait(timeout=150)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)   # the profiler and the program it runs
            proc.wait()
            return None, f"{counter} pass timed out"
        if rc != 0:
            return None, f"{counter} pass exited with {rc}"
        vals = []
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if (r.get("Counter_Name") == counter and r.get("Kernel_Name", "").startswith(kernel)
                        and r.get("Grid_Size") == grid):
                    vals.append(float(r["Counter_Value"]))
        if not vals:
            return None, f"{counter}: no dispatch of {kernel} at grid {grid}"
        return statistics.median(vals), None


def measure_decode_traffic():
    """HBM bytes per launch of the ctx-8192 partial kernel: FETCH_SIZE and WRITE_SIZE medians, each
    scaled by what the same counter reads for a plain 256 MiB device copy. Returns (bytes, note)."""
    dec = ["--only", "decode", "--no-cpu", "--steps", "20", "--warmup", "2"]
    kern, grid = "void it::attn_decode_kernel<1, false, true, true>", str(32768 * 2)
    got = {}
    for key, counter, args, k, g in (("fetch", "FETCH_SIZE", dec, kern, grid),
                                     ("write", "WRITE_SIZE", dec, kern, grid),
                                     ("cal_fetch", "FETCH_SIZE", ["--copy-calibration"], "__amd_rocclr_copyBuffer", "131072"),
                                     ("cal_write", "WRITE_SIZE", ["--copy-calibration"], "__amd_rocclr_copyBuffer", "131072")):
        v, why = pmc_median(counter, args, k, g)
        if v is None or v <= 0:
            return None, why or f"{counter}: zero reading"
        got[key] = v
    fetch = got["fetch"] * COPY_KIB / got["cal_fetch"]
    write = got["write"] * COPY_KIB / got["cal_write"]
    note = (f"rocprofv3 --pmc in this run: FETCH_SIZE {got['fetch']:.1f} KiB x {COPY_KIB / got['cal_fetch']:.3f} + "
            f"WRITE_SIZE {got['write']:.1f} KiB x {COPY_KIB / got['cal_write']:.3f} (factors from a 256 MiB copy)")
    return int(round((fetch + write) * 1024)), note


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="bounded CPU-baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-chunk", type=int, default=0, help="keys per split for decode (0 = library policy)")
    ap.add_argument("--only", choices=["all", "decode", "prefill", "gdn", "prep", "mtp"], default="all",
                    help="run one section only (profiling runs); the JSON line then carries that section's figures")
    ap.add_argument("--no-pmc", action="store_true",
                    help="skip the rocprofv3 --pmc passes that measure roofline.traffic")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 5 plain device copies of 256 MiB (reference reading for the FETCH_SIZE / "
                         "WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (every GPU box here has "
              "one GPU); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from irontimber_amd import ops
    from irontimber_amd._lib import call
    from irontimber_amd.synth import attn_inputs, gdn_inputs, prep_inputs

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": 256 << 20, "copies": 5}))
        return
    stream_of = lambda: torch.cuda.current_stream().cuda_stream
    res = {}
    us_layer = value_gbs = part_gbs = part_us = prefill_tflops = None
    chunk, NSETS, cpu, head_reps = 64, 40, None, 1
    dbytes = decode_bytes(8192)
    scale = 1.0 / 16
    rnd = lambda v, n: None if v is None else round(v, n)
    K, W = args.steps, args.warmup
    # launches per graph for the figures beside the headline: at least 100, so the replay's own
    # launch cost is spread as it is over the headline's >= 100 timed launches
    KM = max(K, 100)

    # ------------------------------------------------------------------ decode attention, ctx 8192
    if args.only in ("all", "decode"):
        ctx = 8192
        q_np, kb, vb = attn_inputs(1, ctx=ctx, nt=4)
        q4 = torch.from_numpy(q_np.reshape(4, -1)).to(dev)
        q1 = q4[3:4].contiguous()
        NSETS = 40
        kc0 = torch.from_numpy(kb.view(np.int16)).to(dev)
        vc0 = torch.from_numpy(vb.view(np.int16)).to(dev)
        kcs = [kc0.clone() for _ in range(NSETS)]
        vcs = [vc0.clone() for _ in range(NSETS)]
        out = torch.empty(4, NH * HD, device=dev)
        # decode split: the library's automatic choice unless --decode-chunk overrides it
        chunk = args.decode_chunk or 64
        part_bytes = ops.attn_scratch_bytes(ctx - 1, 1, NH, NKV, HD, ops.KERNEL_SPLITK, chunk)
        part = torch.empty(max(part_bytes, ops.attn_scratch_bytes(ctx - 4, 4, NH, NKV, HD, ops.KERNEL_SPLITK, 64),
                               ops.attn_scratch_bytes(ctx - 1, 1, NH, NKV, HD, ops.KERNEL_SPLITK, 64)),
                           dtype=torch.uint8, device=dev)
        scale = 1.0 / 16

        def decode_step(i, q=q1, nt=1):
            call("it_attn_f16_ex", q.data_ptr(), NH * 2 * HD, kcs[i % NSETS].data_ptr(), vcs[i % NSETS].data_ptr(), KVD,
                 ctx - nt, HD, NH, NKV, nt, scale, out.data_ptr(), NH * HD, part.data_ptr(), part.numel(),
                 ops.KERNEL_AUTO if nt > 1 or not args.decode_chunk else ops.KERNEL_SPLITK, 0 if nt > 1 else args.decode_chunk,
                 stream_of())

        rec_layout = 1 if 16 < -(-ctx // chunk) <= 256 else 0   # as it_attn_f16 picks for one token
        # the headline layer's partial kernel alone: record layout 1 is the one it_attn_f16 writes for
        # its wave merge (same kernel instantiation as inside decode_step)
        def decode_partials(i):
            call("it_attn_partials_ex", q1.data_ptr(), NH * 2 * HD, kcs[i % NSETS].data_ptr(), vcs[i % NSETS].data_ptr(),
                 KVD, ctx - 1, HD, NH, NKV, 1, scale, part.data_ptr(), part.numel(), chunk, rec_layout, stream_of())

        # correctness guard on the benchmarked path (eager vs graph replays)
        decode_step(0)
        torch.cuda.synchronize()
        ref_out = out[:1].clone()

        # headline: exactly K steps in the timed region (warmup W untimed), graph of K steps
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for i in range(W):
                decode_step(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(K):
                decode_step(i)
        g.replay()   # untimed replay (graph upload)
        torch.cuda.synchronize()
        # the K-step graph is replayed back to back until at least 100 launches sit between the
        # events (one replay when K >= 100), so a short --steps still times >= 100 layers
        head_reps = -(-100 // K)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            e0.record(s)
            for _ in range(head_reps):
                g.replay()
            e1.record(s)
        torch.cuda.synchronize()
        total_ms = e0.elapsed_time(e1)
        assert torch.equal(out[:1], ref_out), "graph replay changed the decode result"
        us_layer = total_ms * 1000.0 / (K * head_reps)
        dbytes = decode_bytes(ctx)
        value_gbs = dbytes / (us_layer * 1e-6) / 1e9
        res["decode_ctx8192_us_per_layer"] = round(us_layer, 3)
        res["decode_ctx8192_GBs"] = round(value_gbs, 1)
        log(f"decode ctx8192: {us_layer:.2f} us/layer, {value_gbs:.0f} GB/s")

        # the same decode layer in one launch through a mailbox (it_attn_f16_mailbox), a named extra
        mbox = ops.attn_mailbox(ctx, 1, NH, dev)

        def decode_one_launch(i):
            call("it_attn_f16_mailbox", q1.data_ptr(), NH * 2 * HD, kcs[i % NSETS].data_ptr(),
                 vcs[i % NSETS].data_ptr(), KVD, ctx - 1, HD, NH, NKV, 1, scale, out.data_ptr(), NH * HD,
                 mbox.data_ptr(), mbox.numel(), part.data_ptr(), part.numel(), stream_of())

        assert ops.attn_mailbox_would_launch(ctx - 1, 1, NH, NKV, mbox)
        decode_one_launch(0)
        torch.cuda.synchronize()
        if not args.decode_chunk:   # same 64-key splits and merge order as the two-launch path
            assert torch.equal(out[:1], ref_out), "one-launch decode differs from the two-launch result"
        ms = graph_time_ms(torch, lambda: [decode_one_launch(i) for i in range(KM)], reps=3)
        assert not ops.attn_mailbox_poisoned(mbox)
        res["decode_ctx8192_one_launch_us_per_layer"] = round(ms * 1000.0 / KM, 3)
        log(f"decode ctx8192 in one launch (mailbox): {ms * 1000.0 / KM:.2f} us/layer")

        # dominant kernel alone: the split-K partial kernel, K launches per graph
        ms_part = graph_time_ms(torch, lambda: [decode_partials(i) for i in range(KM)], reps=3)
        part_us = ms_part * 1000.0 / KM
        part_gbs = dbytes / (part_us * 1e-6) / 1e9
        log(f"decode partial kernel: {part_us:.2f} us, {part_gbs:.0f} GB/s")

        # MTP verify: 4 query positions attending 8189..8192 keys
        ms = graph_time_ms(torch, lambda: [decode_step(i, q4, 4) for i in range(KM)], reps=3)
        res["verify_nt4_us_per_layer"] = round(ms * 1000.0 / KM, 3)
        res["verify_nt4_GBs"] = round(decode_bytes(ctx, 4) / (ms * 1e-3 / KM) / 1e9, 1)

        # decode at ctx 512 (config 1, seed 0)
        q5, kb5, vb5 = attn_inputs(0, ctx=512, nt=1)
        q5 = torch.from_numpy(q5.reshape(1, -1)).to(dev)
        k5 = [torch.from_numpy(kb5.view(np.int16)).to(dev) for _ in range(8)]
        v5 = [torch.from_numpy(vb5.view(np.int16)).to(dev) for _ in range(8)]

        def d512(i):
            # the library's own split (as an engine calls it) unless --decode-chunk fixes one
            call("it_attn_f16_ex", q5.data_ptr(), NH * 2 * HD, k5[i % 8].data_ptr(), v5[i % 8].data_ptr(), KVD, 511, HD,
                 NH, NKV, 1, scale, out.data_ptr(), NH * HD, part.data_ptr(), part.numel(),
                 ops.KERNEL_SPLITK if args.decode_chunk else ops.KERNEL_AUTO, args.decode_chunk, stream_of())
        ms = graph_time_ms(torch, lambda: [d512(i) for i in range(KM)], reps=3)
        res["decode_ctx512_us_per_layer"] = round(ms * 1000.0 / KM, 3)
        del kcs, vcs, k5, v5

    # ------------------------------------------------------------------ prefill attention (config 3)
    mfma_meas = None
    if args.only in ("all", "prefill"):
        # the device's sustained f16 matrix-core rate (it_calib_mfma_f16: MFMA chains, no memory)
        cw, ci = 2048, 2048
        cout = torch.empty(cw * 256, device=dev)
        ms = graph_time_ms(torch, lambda: call("it_calib_mfma_f16", cw, ci, cout.data_ptr(), stream_of()), reps=3)
        mfma_meas = round(cw * 4 * 4 * ci * 32768 / (ms * 1e-3) / 1e12, 1)
        res["mfma_f16_measured_TFLOPs"] = mfma_meas
        log(f"mfma: sustained f16 32x32x16 rate {mfma_meas} TF/s")
        T = 8192
        qp_np, kbp, vbp = attn_inputs(2, ctx=T, nt=T)
        qp = torch.from_numpy(qp_np.reshape(T, -1)).to(dev)
        kp = torch.from_numpy(kbp.view(np.int16)).to(dev)
        vp = torch.from_numpy(vbp.view(np.int16)).to(dev)
        outp = torch.empty(T, NH * HD, device=dev)
        # the chunk calls get exactly the reference engine's arena room for a 64-token chunk at
        # capacity 8192 (attention_dispatch_room, src/vk/mod.rs:148-150): what a drop-in caller passes
        from irontimber_amd._lib import lib as _lr
        room = _lr().it_attention_dispatch_room(T, NH, 64) * 4
        scr = torch.empty(room, dtype=torch.uint8, device=dev)

        def chunk_call(c):
            call("it_attn_f16", qp[c * 64].data_ptr(), NH * 2 * HD, kp.data_ptr(), vp.data_ptr(), KVD, c * 64, HD, NH, NKV,
                 64, scale, outp[c * 64].data_ptr(), NH * HD, scr.data_ptr(), scr.numel(), stream_of())

        ms = graph_time_ms(torch, lambda: chunk_call(64), reps=5)
        f = prefill_flops(4096, 64)
        res["prefill_chunk64_at4096_us"] = round(ms * 1000, 2)
        res["prefill_chunk64_at4096_TFLOPs"] = round(f / (ms * 1e-3) / 1e12, 2)
        # the same chunk as one call of a sequence, as the decode figures are timed: 40 calls per
        # graph replay, each over its own copy of the 4160-position K/V prefix (40 copies, 340 MB,
        # more than the 256 MB MALL, so no call finds its keys left in cache by the one before).
        # The one-call graph above also pays the replay's own launch cost.
        nrot = 40
        kr = [kp[:4160].clone() for _ in range(nrot)]
        vr = [vp[:4160].clone() for _ in range(nrot)]

        def chunk_seq(i):
            call("it_attn_f16", qp[4096].data_ptr(), NH * 2 * HD, kr[i].data_ptr(), vr[i].data_ptr(), KVD, 4096, HD, NH,
                 NKV, 64, scale, outp[4096].data_ptr(), NH * HD, scr.data_ptr(), scr.numel(), stream_of())
        ms = graph_time_ms(torch, lambda: [chunk_seq(i) for i in range(nrot)], reps=3) / nrot
        res["prefill_chunk64_at4096_in_sequence_us"] = round(ms * 1000, 2)
        res["prefill_chunk64_at4096_in_sequence_TFLOPs"] = round(f / (ms * 1e-3) / 1e12, 2)
        del kr, vr
        ms = graph_time_ms(torch, lambda: [chunk_call(c) for c in range(128)], reps=3)
        f = prefill_flops(0, T)
        res["prefill_8192_as_128_chunks_ms"] = round(ms, 3)
        res["prefill_8192_as_128_chunks_TFLOPs"] = round(f / (ms * 1e-3) / 1e12, 2)

        def whole():
            call("it_attn_f16", qp.data_ptr(), NH * 2 * HD, kp.data_ptr(), vp.data_ptr(), KVD, 0, HD, NH, NKV, T, scale,
                 outp.data_ptr(), NH * HD, None, 0, stream_of())
        # one call processes the whole prompt; four back-to-back calls per graph replay amortise the
        # replay's own launch cost, as the decode figure does over its 400 layers
        ms = graph_time_ms(torch, lambda: [whole() for _ in range(4)], reps=3) / 4
        res["prefill_8192_single_call_ms"] = round(ms, 3)
        res["prefill_8192_single_call_TFLOPs"] = round(f / (ms * 1e-3) / 1e12, 2)
        # The same calls with the query operand pre-converted (it_attn_f16_q16): an engine gets q16 from
        # its pre-pass (it_attn_prep_f16_q16, which rewrites q anyway); here it is made once, as that
        # pre-pass makes it: f16(q * (scale * log2 e)) with the product in f32.
        s16 = float(np.float32(np.float32(scale) * np.float32(1.4426950408889634)))
        q16 = (qp.view(T, NH, 2 * HD)[:, :, :HD] * s16).half().contiguous().view(T, NH * HD)

        def chunk_call_q16(c):
            call("it_attn_f16_q16", qp[c * 64].data_ptr(), NH * 2 * HD, q16[c * 64].data_ptr(), NH * HD, kp.data_ptr(),
                 vp.data_ptr(), KVD, c * 64, HD, NH, NKV, 64, scale, outp[c * 64].data_ptr(), NH * HD, scr.data_ptr(),
                 scr.numel(), stream_of())
        ms = graph_time_ms(torch, lambda: [chunk_call_q16(c) for c in range(128)], reps=3)
        res["prefill_8192_as_128_chunks_q16_ms"] = round(ms, 3)
        res["prefill_8192_as_128_chunks_q16_TFLOPs"] = round(f / (ms * 1e-3) / 1e12, 2)

        def whole_q16():
            call("it_attn_f16_q16", qp.data_ptr(), NH * 2 * HD, q16.data_ptr(), NH * HD, kp.data_ptr(), vp.data_ptr(),
                 KVD, 0, HD, NH, NKV, T, scale, outp.data_ptr(), NH * HD, None, 0, stream_of())
        ms = graph_time_ms(torch, lambda: [whole_q16() for _ in range(4)], reps=3) / 4
        res["prefill_8192_single_call_q16_ms"] = round(ms, 3)
        res["prefill_8192_single_call_q16_TFLOPs"] = round(f / (ms * 1e-3) / 1e12, 2)
        log(f"prefill with q16 from the pre-pass: 128 chunks {res['prefill_8192_as_128_chunks_q16_TFLOPs']} TF/s, "
            f"single call {res['prefill_8192_single_call_q16_TFLOPs']} TF/s")
        del q16
        # the configured workload (config 3: the prompt as 128 consecutive 64-token chunks) is the
        # headline; the single whole-prompt call is reported beside it under its own name
        prefill_tflops = res["prefill_8192_as_128_chunks_TFLOPs"]
        log(f"prefill: chunk@4096 {res['prefill_chunk64_at4096_TFLOPs']} TF/s, 128 chunks "
            f"{res['prefill_8192_as_128_chunks_TFLOPs']} TF/s, single call {res['prefill_8192_single_call_TFLOPs']} TF/s")
        del qp, kp, vp, outp, scr

    # ------------------------------------------------------------------ attention pre-pass (norm, rope, KV append)
    if args.only in ("all", "prep"):
        T = 8192
        dp = prep_inputs(7, T)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)
        pq, pk, pv, pqn, pkn = t(dp["q"]), t(dp["k"]), t(dp["v"]), t(dp["q_norm"]), t(dp["k_norm"])
        pkc = torch.empty(T, KVD, dtype=torch.int16, device=dev)
        pvc = torch.empty_like(pkc)

        def prep(nt, pos0):
            ops.attn_prep_f16(pq[:nt], pk[:nt], pv[:nt], pkc, pvc, pos0, NH, NKV, pqn, pkn)
        ms = graph_time_ms(torch, lambda: [prep(1, T - 1) for _ in range(KM)], reps=3)
        res["prep_decode_us"] = round(ms * 1000 / KM, 3)
        ms = graph_time_ms(torch, lambda: [prep(64, 4096) for _ in range(100)], reps=3)
        res["prep_chunk64_us"] = round(ms * 10, 3)
        ms = graph_time_ms(torch, lambda: [prep(T, 0) for _ in range(10)], reps=3)
        ms /= 10
        res["prep_8192_us"] = round(ms * 1000, 2)
        res["prep_8192_GBs"] = round(prep_bytes(T) / (ms * 1e-3) / 1e9, 1)
        log(f"prep: decode {res['prep_decode_us']} us, chunk64 {res['prep_chunk64_us']} us, 8192 tokens "
            f"{res['prep_8192_us']} us ({res['prep_8192_GBs']} GB/s)")
        del pq, pk, pv, pkc, pvc

    # ------------------------------------------------------------------ MTP head: f32-KV attention
    if args.only in ("all", "mtp"):
        S8 = 8192
        NMT = 12   # 12 f32 caches of 32 MiB: 384 MiB rotated, beyond the 256 MB MALL
        g = torch.Generator(device=dev).manual_seed(5)
        kf = [torch.randn(S8, KVD, device=dev, generator=g) for _ in range(NMT)]
        vf = [torch.randn(S8, KVD, device=dev, generator=g) for _ in range(NMT)]
        qm = torch.randn(64, NH * 2 * HD, device=dev, generator=g)
        om = torch.empty(64, NH * HD, device=dev)
        from irontimber_amd._lib import lib as _lm
        scm = torch.empty(max(_lm().it_attn_f32kv_scratch_bytes(p0, n, HD, NH, NKV)
                              for p0, n in ((S8 - 1, 1), (S8 - 2, 2), (1024, 64), (2048, 64), (4096, 64), (S8 - 64, 64))),
                          dtype=torch.uint8, device=dev)

        def mtp_attn(i, nt, pos0):
            call("it_attn_f32kv", qm.data_ptr(), NH * 2 * HD, kf[i % NMT].data_ptr(), vf[i % NMT].data_ptr(), KVD, pos0,
                 HD, NH, NKV, nt, scale, om.data_ptr(), NH * HD, scm.data_ptr(), scm.numel(), stream_of())
        ms = graph_time_ms(torch, lambda: [mtp_attn(i, 1, S8 - 1) for i in range(KM)], reps=3)
        us = ms * 1000 / KM
        fb = 2 * S8 * KVD * 4 + NH * 2 * HD * 4 + NH * HD * 4
        res["mtp_f32kv_decode_8192_us"] = round(us, 3)
        res["mtp_f32kv_decode_8192_GBs"] = round(fb / (us * 1e-6) / 1e9, 1)
        ms = graph_time_ms(torch, lambda: [mtp_attn(i, 2, S8 - 2) for i in range(KM)], reps=3)
        res["mtp_f32kv_nt2_8192_us"] = round(ms * 1000 / KM, 3)
        ms = graph_time_ms(torch, lambda: [mtp_attn(i, 64, 4096) for i in range(20)], reps=3)
        res["mtp_f32kv_catchup64_at4096_us"] = round(ms * 1000 / 20, 2)
        for p0 in (1024, 2048, S8 - 64):   # the catch-up at other prompt positions
            ms = graph_time_ms(torch, lambda: [mtp_attn(i, 64, p0) for i in range(20)], reps=3)
            res[f"mtp_f32kv_catchup64_at{p0}_us"] = round(ms * 1000 / 20, 2)
        # the same catch-up given exactly the reference arena's room (src/vk/mod.rs:148, 730-733):
        # the library's preferred split fits it (64-key splits would not)
        room = _lm().it_attention_dispatch_room(S8, NH, 64) * 4
        scr_room = torch.empty(room, dtype=torch.uint8, device=dev)

        def mtp_room(i):
            call("it_attn_f32kv", qm.data_ptr(), NH * 2 * HD, kf[i % NMT].data_ptr(), vf[i % NMT].data_ptr(), KVD,
                 4096, HD, NH, NKV, 64, scale, om.data_ptr(), NH * HD, scr_room.data_ptr(), room, stream_of())
        ms = graph_time_ms(torch, lambda: [mtp_room(i) for i in range(20)], reps=3)
        res["mtp_f32kv_catchup64_at4096_room_us"] = round(ms * 1000 / 20, 2)
        log(f"mtp f32-KV attention: decode 8192 slots {res['mtp_f32kv_decode_8192_us']} us "
            f"({res['mtp_f32kv_decode_8192_GBs']} GB/s), nt=2 {res['mtp_f32kv_nt2_8192_us']} us, "
            f"64-token catch-up at 4096 {res['mtp_f32kv_catchup64_at4096_us']} us, "
            f"{res['mtp_f32kv_catchup64_at4096_room_us']} us within the reference room; at 1024 / 2048 / "
            f"{S8 - 64}: {res['mtp_f32kv_catchup64_at1024_us']} / {res['mtp_f32kv_catchup64_at2048_us']} / "
            f"{res[f'mtp_f32kv_catchup64_at{S8 - 64}_us']} us")
        del scr_room
        del kf, vf, scm

    # ------------------------------------------------------------------ GDN decode step (config 4)
    if args.only in ("all", "gdn"):
        nv, nk, S = 32, 16, 128
        d = gdn_inputs(3, nt=1, nv=nv, nk=nk)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)
        NST = 160
        states = [t(d["state"]) for _ in range(NST)]
        x, w, cst = t(d["x"]), t(d["w"]), t(d["conv_state"])
        br, ar, dtv, av = t(d["beta_raw"]), t(d["alpha_raw"]), t(d["dt"]), t(d["a"])
        co = torch.empty(1, d["cd"], device=dev)
        og = torch.empty(1, nv * S, device=dev)

        def gdn_layer(i):
            call("it_gdn_conv_l2norm", x.data_ptr(), d["cd"], w.data_ptr(), cst.data_ptr(), co.data_ptr(), d["cd"],
                 d["cd"], 1, 4, 2 * nk, 1e-6, stream_of())
            call("it_gdn_step", co.data_ptr(), d["cd"], br.data_ptr(), ar.data_ptr(), nv, dtv.data_ptr(), av.data_ptr(),
                 states[i % NST].data_ptr(), og.data_ptr(), nv * S, 1, nv, nk, S, stream_of())

        def gdn_only(i):
            call("it_gdn_step", co.data_ptr(), d["cd"], br.data_ptr(), ar.data_ptr(), nv, dtv.data_ptr(), av.data_ptr(),
                 states[i % NST].data_ptr(), og.data_ptr(), nv * S, 1, nv, nk, S, stream_of())
        ms = graph_time_ms(torch, lambda: [gdn_layer(i) for i in range(KM)], reps=3)
        res["gdn_decode_layer_us"] = round(ms * 1000 / KM, 3)
        ms = graph_time_ms(torch, lambda: [gdn_only(i) for i in range(KM)], reps=3)
        gst_us = ms * 1000 / KM
        gbytes = 2 * nv * S * S * 4
        res["gdn_step_us"] = round(gst_us, 3)
        res["gdn_step_state_GBs"] = round(gbytes / (gst_us * 1e-6) / 1e9, 1)
        log(f"gdn: layer {res['gdn_decode_layer_us']} us, step {gst_us:.2f} us ({res['gdn_step_state_GBs']} GB/s state)")

        # the same layer in one launch (conv state ping-pongs between two buffers)
        cst2 = [t(d["conv_state"]), t(d["conv_state"])]

        def gdn_layer_fused(i):
            call("it_gdn_decode_fused", x.data_ptr(), d["cd"], w.data_ptr(), 4, cst2[i & 1].data_ptr(),
                 cst2[(i + 1) & 1].data_ptr(), br.data_ptr(), ar.data_ptr(), nv, dtv.data_ptr(), av.data_ptr(),
                 states[i % NST].data_ptr(), og.data_ptr(), nv * S, 1, nv, nk, S, 1e-6, stream_of())
        ms = graph_time_ms(torch, lambda: [gdn_layer_fused(i) for i in range(KM)], reps=3)
        res["gdn_decode_layer_fused_us"] = round(ms * 1000 / KM, 3)
        log(f"gdn: layer in one launch {res['gdn_decode_layer_fused_us']} us")

        # the reference's whole GDN decode output: recurrence + gated RMSNorm (rmsnorm mode 1), as two
        # kernels and as one (the per-head recurrence with the epilogue fused)
        zg = torch.randn(1, nv * S, device=dev)
        nwg = torch.ones(S, device=dev)
        og2g = torch.empty(1, nv * S, device=dev)

        def gdn_gated_two(i):
            gdn_only(i)
            call("it_gdn_gated_rmsnorm", og.data_ptr(), nv * S, zg.data_ptr(), nv * S, nwg.data_ptr(), 1e-6,
                 og2g.data_ptr(), nv * S, nv, S, 1, stream_of())

        def gdn_head(i, gated):
            call("it_gdn_step_gated", co.data_ptr(), d["cd"], br.data_ptr(), ar.data_ptr(), nv, dtv.data_ptr(),
                 av.data_ptr(), states[i % NST].data_ptr(), og2g.data_ptr(), nv * S, 1, nv, nk, S,
                 zg.data_ptr() if gated else None, nv * S, nwg.data_ptr(), 1e-6, None, 0, stream_of())
        ms = graph_time_ms(torch, lambda: [gdn_gated_two(i) for i in range(KM)], reps=3)
        res["gdn_step_plus_gated_norm_two_kernels_us"] = round(ms * 1000 / KM, 3)
        ms = graph_time_ms(torch, lambda: [gdn_head(i, False) for i in range(KM)], reps=3)
        res["gdn_step_head_kernel_us"] = round(ms * 1000 / KM, 3)
        ms = graph_time_ms(torch, lambda: [gdn_head(i, True) for i in range(KM)], reps=3)
        res["gdn_step_gated_fused_us"] = round(ms * 1000 / KM, 3)

        def gdn_layer_gated(i):
            call("it_gdn_conv_l2norm", x.data_ptr(), d["cd"], w.data_ptr(), cst.data_ptr(), co.data_ptr(), d["cd"],
                 d["cd"], 1, 4, 2 * nk, 1e-6, stream_of())
            gdn_head(i, True)
        ms = graph_time_ms(torch, lambda: [gdn_layer_gated(i) for i in range(KM)], reps=3)
        res["gdn_decode_layer_gated_us"] = round(ms * 1000 / KM, 3)
        log(f"gdn: step + gated norm as two kernels {res['gdn_step_plus_gated_norm_two_kernels_us']} us, "
            f"per-head step {res['gdn_step_head_kernel_us']} us, fused gated {res['gdn_step_gated_fused_us']} us; "
            f"layer with the gated output {res['gdn_decode_layer_gated_us']} us")

        # MTP verify of [x, draft]: one nt = 2 layer call with the conv and SSM checkpoints after token 0
        d2 = gdn_inputs(3, nt=2, nv=nv, nk=nk)
        x2, br2, ar2 = t(d2["x"]), t(d2["beta_raw"]), t(d2["alpha_raw"])
        co2, og2 = torch.empty(2, d["cd"], device=dev), torch.empty(2, nv * S, device=dev)
        ck_conv, ck_ssm = torch.empty_like(cst), torch.empty_like(states[0])

        def gdn_verify(i):
            call("it_gdn_conv_l2norm_ckpt", x2.data_ptr(), d["cd"], w.data_ptr(), cst.data_ptr(), co2.data_ptr(),
                 d["cd"], d["cd"], 2, 4, 2 * nk, 1e-6, ck_conv.data_ptr(), 0, stream_of())
            call("it_gdn_step_ckpt", co2.data_ptr(), d["cd"], br2.data_ptr(), ar2.data_ptr(), nv, dtv.data_ptr(),
                 av.data_ptr(), states[i % NST].data_ptr(), og2.data_ptr(), nv * S, 2, nv, nk, S, ck_ssm.data_ptr(), 0,
                 stream_of())
        ms = graph_time_ms(torch, lambda: [gdn_verify(i) for i in range(KM)], reps=3)
        res["gdn_verify_nt2_layer_us"] = round(ms * 1000 / KM, 3)

        def gdn_verify_fused(i):
            call("it_gdn_decode_fused_ckpt", x2.data_ptr(), d["cd"], w.data_ptr(), 4, cst2[i & 1].data_ptr(),
                 cst2[(i + 1) & 1].data_ptr(), br2.data_ptr(), ar2.data_ptr(), nv, dtv.data_ptr(), av.data_ptr(),
                 states[i % NST].data_ptr(), og2.data_ptr(), nv * S, 2, nv, nk, S, 1e-6, ck_ssm.data_ptr(),
                 ck_conv.data_ptr(), 0, stream_of())
        ms = graph_time_ms(torch, lambda: [gdn_verify_fused(i) for i in range(KM)], reps=3)
        res["gdn_verify_nt2_layer_fused_us"] = round(ms * 1000 / KM, 3)

        def gdn_reject(i):
            call("it_gdn_rollback", ck_conv.data_ptr(), cst.data_ptr(), cst.numel(), ck_ssm.data_ptr(),
                 states[i % NST].data_ptr(), ck_ssm.numel(), stream_of())
        ms = graph_time_ms(torch, lambda: [gdn_reject(i) for i in range(KM)], reps=3)
        res["gdn_rollback_us"] = round(ms * 1000 / KM, 3)
        log(f"gdn verify nt=2 layer (with checkpoints) {res['gdn_verify_nt2_layer_us']} us, "
            f"in one launch {res['gdn_verify_nt2_layer_fused_us']} us, rollback {res['gdn_rollback_us']} us")
        del states

        # ------------------------------------------------------------------ GDN chunked prefill (config 5)
        T5 = 8192
        d5 = gdn_inputs(4, nt=T5, nv=nv, nk=nk)
        x5, w5, cs5 = t(d5["x"]), t(d5["w"]), t(d5["conv_state"])
        br5, ar5, dt5, a5 = t(d5["beta_raw"]), t(d5["alpha_raw"]), t(d5["dt"]), t(d5["a"])
        st5 = t(d5["state"])
        co5 = torch.empty(T5, d5["cd"], device=dev)
        o5 = torch.empty(T5, nv * S, device=dev)
        from irontimber_amd._lib import lib as _l
        scr5 = torch.empty(_l().it_gdn_chunked_scratch_bytes(T5, nv, S), dtype=torch.uint8, device=dev)

        def gdn_prefill():
            call("it_gdn_conv_l2norm", x5.data_ptr(), d5["cd"], w5.data_ptr(), cs5.data_ptr(), co5.data_ptr(), d5["cd"],
                 d5["cd"], T5, 4, 2 * nk, 1e-6, stream_of())
            call("it_gdn_chunked", co5.data_ptr(), d5["cd"], br5.data_ptr(), ar5.data_ptr(), nv, dt5.data_ptr(),
                 a5.data_ptr(), st5.data_ptr(), o5.data_ptr(), nv * S, T5, nv, nk, S, scr5.data_ptr(), scr5.numel(),
                 stream_of())

        def gdn_scan_only():
            call("it_gdn_chunked", co5.data_ptr(), d5["cd"], br5.data_ptr(), ar5.data_ptr(), nv, dt5.data_ptr(),
                 a5.data_ptr(), st5.data_ptr(), o5.data_ptr(), nv * S, T5, nv, nk, S, scr5.data_ptr(), scr5.numel(),
                 stream_of())
        ms = graph_time_ms(torch, gdn_prefill, reps=3)
        res["gdn_prefill_8192_layer_ms"] = round(ms, 4)
        ms_s = graph_time_ms(torch, gdn_scan_only, reps=3)
        gflop = 47.96e9   # chunked-form flops for 8192 tokens, 32 V heads, C=64
        res["gdn_prefill_8192_scan_ms"] = round(ms_s, 4)
        res["gdn_prefill_8192_scan_TFLOPs"] = round(gflop / (ms_s * 1e-3) / 1e12, 2)
        io = T5 * (2 * nk + nv) * S * 4 + T5 * nv * S * 4 + 2 * 2 * nv * S * S * 4 + 2 * T5 * nv * 4
        res["gdn_prefill_8192_scan_io_GBs"] = round(io / (ms_s * 1e-3) / 1e9, 1)
        log(f"gdn prefill 8192: layer {ms:.3f} ms, scan {ms_s:.3f} ms ({res['gdn_prefill_8192_scan_TFLOPs']} TF/s chunked)")
        # the same layer in one call, the conv output kept as f16 (config 5's f16 activations)
        scr1 = torch.empty(_l().it_gdn_prefill_scratch_bytes(T5, nv, nk, S), device=dev, dtype=torch.uint8)

        def gdn_prefill_one():
            call("it_gdn_prefill", x5.data_ptr(), d5["cd"], w5.data_ptr(), 4, cs5.data_ptr(), br5.data_ptr(),
                 ar5.data_ptr(), nv, dt5.data_ptr(), a5.data_ptr(), st5.data_ptr(), o5.data_ptr(), nv * S, T5, nv,
                 nk, S, 1e-6, scr1.data_ptr(), scr1.numel(), stream_of())
        ms1 = graph_time_ms(torch, gdn_prefill_one, reps=3)
        res["gdn_prefill_8192_layer_one_call_ms"] = round(ms1, 4)
        log(f"gdn prefill 8192 in one call (f16 conv output): layer {ms1:.3f} ms")
        z5 = torch.randn(T5, nv * S, device=dev)
        nw5 = torch.ones(S, device=dev)

        def gated5():
            call("it_gdn_gated_rmsnorm", o5.data_ptr(), nv * S, z5.data_ptr(), nv * S, nw5.data_ptr(), 1e-6,
                 o5.data_ptr(), nv * S, nv, S, T5, stream_of())
        ms_g = graph_time_ms(torch, lambda: [gated5() for _ in range(10)], reps=3) / 10
        res["gdn_prefill_8192_gated_norm_us"] = round(ms_g * 1000, 2)
        res["gdn_prefill_8192_gated_norm_GBs"] = round(3 * T5 * nv * S * 4 / (ms_g * 1e-3) / 1e9, 1)
        log(f"gdn prefill gated norm: {res['gdn_prefill_8192_gated_norm_us']} us "
            f"({res['gdn_prefill_8192_gated_norm_GBs']} GB/s)")
        del z5

        # hybrid stack (config 5): 3 GDN prefill layers then 1 attention prefill layer, 8192 tokens
        T = 8192
        qp_np, kbp, vbp = attn_inputs(2, ctx=T, nt=T)
        qp = torch.from_numpy(qp_np.reshape(T, -1)).to(dev)
        kp = torch.from_numpy(kbp.view(np.int16)).to(dev)
        vp = torch.from_numpy(vbp.view(np.int16)).to(dev)
        outp = torch.empty(T, NH * HD, device=dev)

        def hybrid():   # each GDN layer in one call (it_gdn_prefill)
            for _ in range(3):
                gdn_prefill_one()
            call("it_attn_f16", qp.data_ptr(), NH * 2 * HD, kp.data_ptr(), vp.data_ptr(), KVD, 0, HD, NH, NKV, T, scale,
                 outp.data_ptr(), NH * HD, None, 0, stream_of())
        ms = graph_time_ms(torch, hybrid, reps=2)
        res["hybrid_3gdn_1attn_prefill_8192_ms"] = round(ms, 3)
        log(f"hybrid 3 GDN + 1 attention prefill layers, 8192 tokens: {ms:.3f} ms")
        del qp, kp, vp, outp, co5, o5, scr5, scr1

    # ------------------------------------------------------------------ CPU baselines (oracle, host cores)
    # The C++ restatement of src/cpu.rs timed on this box's host cores, one bounded sample per
    # configuration. Threads: the CPU share of a one-GPU box (16), which is below the host's
    # hardware_concurrency(); both numbers are reported.
    cpu_all = {}
    if args.only == "all" and not args.no_cpu:
        import oracle
        hw = oracle.hardware_threads()
        threads = min(16, hw)
        per = args.cpu_seconds / 4

        def timed(fn, cap=100000):
            n, t0 = 0, time.perf_counter()
            while True:
                fn()
                n += 1
                el = time.perf_counter() - t0
                if el >= per or n >= cap:
                    return n, el
        # config 2: one decode-attention layer at ctx 8192
        q2, kb2, vb2 = attn_inputs(1, ctx=8192, nt=1)
        n, el = timed(lambda: oracle.attn(q2.reshape(1, -1), kb2, vb2, 8191, NH, NKV, threads=threads))
        us = el / n * 1e6
        cpu_all["config2_decode_ctx8192"] = {"us_per_layer": round(us, 1), "GBs": round(decode_bytes(8192) / us / 1e3, 2),
                                             "sample": f"{n} layers, {el:.1f} s"}
        # config 3(i): one 64-token chunk after 4096 cached positions
        q3, kb3, vb3 = attn_inputs(2, ctx=4096 + 64, nt=64)
        n, el = timed(lambda: oracle.attn(q3.reshape(64, -1), kb3, vb3, 4096, NH, NKV, threads=threads))
        us = el / n * 1e6
        cpu_all["config3_chunk64_at4096"] = {"us": round(us, 1), "TFLOPs": round(prefill_flops(4096, 64) / us / 1e6, 4),
                                             "sample": f"{n} chunks, {el:.1f} s"}
        # config 4: the GDN decode layer (conv + L2 + recurrence), one token
        d4 = gdn_inputs(3, nt=1)
        cs4, st4 = d4["conv_state"].copy(), d4["state"].copy()
        o4, c4 = np.zeros((1, 32 * 128), np.float32), np.zeros((1, d4["cd"]), np.float32)
        P = lambda a: a.ctypes.data
        L = oracle.lib()

        def gdn_tokens(d, cs, st, o, c, nt):
            L.it_ref_gdn_layer(P(d["x"]), d["cd"], P(d["w"]), P(cs), 4, P(d["beta_raw"]), P(d["alpha_raw"]), 32,
                               P(d["dt"]), P(d["a"]), P(st), P(o), 32 * 128, P(c), nt, 32, 16, 128, 1e-6, threads)
        n, el = timed(lambda: gdn_tokens(d4, cs4, st4, o4, c4, 1))
        us = el / n * 1e6
        cpu_all["config4_gdn_decode_layer"] = {"us_per_layer": round(us, 1),
                                               "state_GBs": round(2 * 32 * 128 * 128 * 4 / us / 1e3, 2),
                                               "sample": f"{n} tokens, {el:.1f} s"}
        # config 5: the GDN prefill over 8192 tokens, token-sequential as cpu.rs runs it; a bounded
        # prefix of the prompt is timed and scaled to 8192 tokens (per-token cost is constant)
        T5c = 256
        d5c = gdn_inputs(4, nt=T5c)
        cs5c, st5c = d5c["conv_state"].copy(), d5c["state"].copy()
        o5c, c5c = np.zeros((T5c, 32 * 128), np.float32), np.zeros((T5c, d5c["cd"]), np.float32)
        n, el = timed(lambda: gdn_tokens(d5c, cs5c, st5c, o5c, c5c, T5c), cap=50)
        ms_tok = el / n / T5c * 1e3
        cpu_all["config5_gdn_prefill_8192"] = {"ms": round(ms_tok * 8192, 2), "ms_per_token": round(ms_tok, 4),
                                               "sample": f"{n} x {T5c}-token prefixes, {el:.1f} s, scaled to 8192"}
        us2 = cpu_all["config2_decode_ctx8192"]["us_per_layer"]
        cpu = {"value": cpu_all["config2_decode_ctx8192"]["GBs"], "unit": "GB/s", "cores": threads,
               "hardware_threads": hw, "kind": "port", "us_per_layer": us2,
               "sample": f"config 2: {cpu_all['config2_decode_ctx8192']['sample']} of decode attention at ctx 8192 "
                         f"through oracle/cpu_ref.cpp (restatement of src/cpu.rs:243-274), {threads} threads "
                         f"(the one-GPU box's CPU share; hardware_concurrency {hw})",
               "configs": cpu_all}
        log(f"cpu baselines ({threads} threads of {hw}): " + json.dumps(cpu_all))

    traffic, traffic_note = None, "not measured (--no-pmc or a section run)"
    if args.only == "all" and not args.no_pmc and us_layer is not None:
        log("roofline.traffic: four rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE; decode and a copy)")
        traffic, traffic_note = measure_decode_traffic()
        log(f"traffic: {traffic} bytes per launch ({traffic_note})")
    line = {
        "metric": "decode attn µs/layer + HBM GB/s @ctx 8192; prefill attn TFLOP/s @8192 tok",
        "value": rnd(value_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": rnd(None if us_layer is None else us_layer / 1000.0, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded splitmix64 N(0,1), BASELINE configs 1-4)",
        "config": {"workload": "decode attention, 1 layer, batch 1, 16 q / 2 KV heads, head_dim 256, "
                               "f16 KV cache 8192 positions (config 2, seed 1)",
                   "kv_rotation_sets": NSETS, "split_keys": chunk,
                   "timing": (f"hip events around {head_reps} back-to-back replay(s) of a graph of the {K} timed "
                              f"layers ({K * head_reps} launches of it_attn_f16 timed; value per layer)"
                              if us_layer is not None else "hip graph replay, hip events")},
        "decode_us_per_layer": rnd(us_layer, 3),
        "prefill_attn_TFLOPs": prefill_tflops,
        "results": res,
        "roofline": {"bound": "hbm", "achieved": rnd(part_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": rnd(None if part_gbs is None else part_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_unit": "bytes per launch", "traffic_source": traffic_note,
                     "kernel": "attn_decode_kernel<1, false, true, true>", "kernel_us": rnd(part_us, 3),
                     "bytes_per_launch": dbytes},
        "roofline_prefill": {"bound": "mfma", "achieved": prefill_tflops, "peak": F16_MFMA_PEAK_TFLOPS,
                             "unit": "TFLOP/s", "frac": rnd(None if prefill_tflops is None else prefill_tflops / F16_MFMA_PEAK_TFLOPS, 4),
                             "measured_peak": mfma_meas,
                             "frac_of_measured": rnd(None if prefill_tflops is None or not mfma_meas
                                                     else prefill_tflops / mfma_meas, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
