#!/usr/bin/env python3
"""bench.py - batch-1 decode tokens/s (+ % of HBM peak) and prefill tokens/s of the 8B-shape q8 Llama on one MI355X.

Workload (the C3 / C4 benchmark configurations): Llama-3-8B shape (32 layers, hidden 4096, 32 / 8 heads, head_dim 128,
SwiGLU 14336, vocab 128256, untied head), seeded N(0, 0.02) random-init weights in q8, fp16 KV cache.
  decode  - 128-token prompt, `--warmup` untimed greedy tokens, then exactly `--steps` greedy tokens timed (device
            argmax feeds the next step; HIP events on the model's stream, host clock around it)
  prefill - one `--prefill-tokens` prompt (C4), host clock around qph_prefill
Roofline: the dominant decode kernel (fused RMSNorm + gate/up + SwiGLU matvec, ~47 % of the step's bytes) in the form
the token loop runs it at the timed contexts (PRO_NORM: the fused attention + wo kernel has already added its kv-group
partials to the residual stream; with QPH_AWO_SUM=0 this kernel adds them, PRO_NORM_SUM) launched alone over the 32
layers in turn and timed with HIP events on the model's stream; achieved = its algorithmic bytes / mean duration.  traffic = its HBM bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE (committed summary under
profiles/, produced by --profile runs and --pmc-summary).
CPU baseline: the reference engine compiled from its own sources (oracle/_ref/libqpref.so, AVX2) on the same file,
on the host cores, qpack-bench protocol on a bounded sample.

Prints ONE JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import sys
import subprocess
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# the token loop's gate / up kernel: PRO_NORM, or PRO_NORM_SUM (QPH_AWO_SUM=0: it adds the fused attention + wo
# kernel's group partials); EPI_SWIGLU, 2 rows per
# unit, q8 - its rocprofv3 name, time_kernel id and the committed counter summary
DOMINANT = {"sum": ("k_matvec<2, 2, 2, 1, false>", 7, "k_matvec_normsum_swiglu_q8_c3_traffic.md",
                    "k_matvec<PRO_NORM_SUM,EPI_SWIGLU> (x + the 8 kv-group partials of the fused attention + wo, "
                    "RMSNorm, gate/up, SwiGLU; 2 x 14336 x 4096 q8; launches walk the 32 layers)"),
            "norm": ("k_matvec<1, 2, 2, 1, false>", 0, "k_matvec_norm_swiglu_q8_c3_traffic.md",
                     "k_matvec<PRO_NORM,EPI_SWIGLU> (fused RMSNorm + gate/up + SwiGLU, 2 x 14336 x 4096 q8; launches "
                     "walk the 32 layers)")}
COPY_BYTES = 1 << 29                         # calibration copy: 512 MiB read + 512 MiB written
METRIC = "batch-1 decode tokens/s + % HBM peak; prefill tokens/s (8B-shape q8)"


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def quant_name(shape):
    if shape.mlp_q1:
        return "q1m" if shape.more_bits else "q1"
    if shape.q4:
        return "q4m" if (shape.q4m_alt or shape.more_bits) else "q4"
    return "q8"


def file_weight_bytes(path):
    """HBM bytes one decode step reads from the weights of a QPACK2 file: every tensor's blobs (data + scale) once,
    except the embedding, of which one row is read - unless it is tied, when it is also the output head"""
    import struct
    with open(path, "rb") as f:
        head = f.read(16)
        n = struct.unpack("<I", head[8:12])[0]
        toc = {}
        for _ in range(n):
            e = f.read(72)
            toc[e[:56].rstrip(b"\0").decode()] = struct.unpack("<QQ", e[56:72])
        off, ln = toc["manifest.json"]
        f.seek(off)
        man = json.loads(f.read(ln))
        f.seek(toc["config.json"][0])
        cfg = json.loads(f.read(toc["config.json"][1]))
    total = 0
    for e in man["tensors"]:
        b = toc[e["blob"]][1] + (toc[e["scale"]][1] if "scale" in e else 0)
        if e["name"] == "embed":
            b = b if cfg.get("tie_embeddings") else b // e["shape"][0]
        total += b
    return total


def step_bytes(weight_bytes, shape, T):
    """algorithmic HBM bytes of one decode step at context T: the weights (file_weight_bytes) and the fp16 K and V rows
    of positions [0, T) in every layer"""
    kvd = shape.kv_heads * shape.head_dim
    return weight_bytes + shape.layers * 2 * T * kvd * 2


def calibration_copy(reps=4):
    """the library's plain copy kernel k_copy over COPY_BYTES (read once, written once) for scaling the byte counters"""
    import qpack_amd as qa
    ms = qa.time_copy(COPY_BYTES, reps)
    log(f"calibration copy: {COPY_BYTES >> 20} MiB in {ms * 1e3:.1f} us -> {2 * COPY_BYTES / (ms / 1e3) / 1e9:.0f} GB/s (read + write)")


def pmc_summary(csv_path, kernel_sub, copy_sub="k_copy"):
    """per-dispatch averages of each counter in a rocprofv3 counter_collection.csv, for the dominant kernel and for the
    calibration copy; returns {counter: (kernel_mean, copy_mean, n_kernel, n_copy)}"""
    import csv
    acc = {}
    with open(csv_path) as f:
        for r in csv.DictReader(f):
            name, ctr, val = r["Kernel_Name"], r["Counter_Name"], float(r["Counter_Value"])
            which = 0 if kernel_sub in name else (1 if copy_sub in name else None)
            if which is None:
                continue
            e = acc.setdefault(ctr, [[], []])
            e[which].append(val)
    return {c: (float(np.mean(k)) if k else None, float(np.mean(cp)) if cp else None, len(k), len(cp))
            for c, (k, cp) in acc.items()}


def read_traffic(name):
    """HBM bytes per launch of the dominant kernel, from the committed counter summary (line 'traffic_bytes: N')"""
    try:
        with open(os.path.join(ROOT, "profiles", name)) as f:
            for line in f:
                if line.startswith("traffic_bytes:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def other_config(name, seed, steps_override=None):
    """decode tokens/s of another benchmark configuration on its own workload: C1 / C2 prompt + greedy tokens (prompt through
    the product's prefill), C5 greedy tokens after restoring a 16384-position N(0, 1) context"""
    import qpack_amd as qa
    shape = qa.CONFIGS[name]
    runs = {"c1": (32, 128, None), "c2": (512, 256, None), "c5": (0, 128, 16384)}
    prompt, steps, restore = runs[name]
    prefill_s = None
    steps = steps_override or steps
    tmpdir = tempfile.mkdtemp(prefix="qpack_bench_")
    path = os.path.join(tmpdir, name + ".qpack")
    try:
        qa.write_synthetic(name, path, seed=seed, threads=min(16, os.cpu_count() or 8))
        wbytes = file_weight_bytes(path)
        ctx = max(prompt, restore or 0) + steps + 16
        m = qa.HipLlama.load(path, max_ctx=ctx)
        rng = np.random.default_rng(seed)
        if restore:
            m.restore(qa.kv_fill_snapshot(shape, restore, seed))
            tok = 1
        else:
            ptoks = rng.integers(0, shape.vocab, prompt).astype(np.int32)
            m.prefill(ptoks, 1)             # warm-up: first launches of the prompt kernels
            m.reset()
            t0 = time.perf_counter()
            lg = m.prefill(ptoks, 1)
            prefill_s = time.perf_counter() - t0
            tok = int(np.argmax(lg))
        T0 = m.pos()
        tok = int(m.greedy_run(tok, 4)[-1])   # warm-up
        T1 = m.pos()
        ms = m.time_greedy(tok, steps)
        att_ms, att_b = m.time_kernel(5, 50)
        m.close()
    finally:
        if os.path.exists(path):
            os.remove(path)
        os.rmdir(tmpdir)
    T2 = T1 + steps
    sb = step_bytes(wbytes, shape, (T1 + 1 + T2) / 2)
    gbs = sb / (ms / 1e3 / steps) / 1e9
    kind = quant_name(shape)
    ctx_desc = f"restored N(0,1) fp16 context of {restore}" if restore else f"{prompt}-token prompt"
    return dict(tokens_per_s=round(steps / (ms / 1e3), 1), ms_per_token=round(ms / steps, 4),
                hbm_pct_of_peak=round(100 * gbs / HBM_PEAK_GBS, 2), bytes_per_token=round(sb),
                attention_us=round(att_ms * 1e3, 2),
                prompt_tokens_per_s=round(prompt / prefill_s, 1) if prefill_s else None,
                workload=f"{name} ({kind}, {shape.layers} layers, hidden {shape.hidden}): {ctx_desc}, 4 warm-up + {steps} "
                         f"timed greedy tokens (context {T1}..{T2})")


REF_BENCH = os.path.join(ROOT, "qpack_amd", "integration", "_build", "qpack-bench")


def cpu_baseline(path, threads):
    """the reference's qpack-bench (tools/qpack-bench.cpp, AVX2 engine, compiled from its sources with the HIP adapter
    linked in but not selected: QPACK_DEVICE unset) on the same C3 file, with its own protocol (:35-62): one child
    process per thread count, prefill np then np decode steps, best of 2 repetitions.  Two rows: min(16, cores) threads
    on the C3 workload's 128-token prompt + 32 decode steps, and 1 thread on a bounded sample (32-token prompt + 8
    steps; the 128-token prompt alone takes ~30 s on one core).  value = the min(16, cores)-thread decode rate."""
    env = dict(os.environ)
    env.pop("QPACK_DEVICE", None)
    rows = []
    for t, np_, ng in ((threads, 128, 32), (1, 32, 8)):
        r = subprocess.run([REF_BENCH, "-m", path, "-p", str(np_), "-n", str(ng), "-t", str(t), "-r", "2"], env=env,
                           capture_output=True, text=True, timeout=900, check=True)
        line = [x for x in r.stdout.splitlines() if x.startswith("|") and not x.startswith("| model") and "---" not in x][0]
        c = [x.strip() for x in line.strip().strip("|").split("|")]
        rows.append(dict(threads=int(c[3]), prompt=np_, decode_steps=ng, prefill_tokens_per_s=float(c[4]),
                         decode_tokens_per_s=float(c[5])))
    top = rows[0]
    return dict(value=top["decode_tokens_per_s"], unit="tokens/s", cores=top["threads"], kind="reference",
                sample=f"reference qpack-bench (AVX2) on the same C3 file: {top['threads']} threads, {top['prompt']}-token "
                       f"prompt + {top['decode_steps']} decode steps, best of 2 (prefill {top['prefill_tokens_per_s']} tok/s); "
                       f"1 thread: {rows[1]['prefill_tokens_per_s']} tok/s prefill, {rows[1]['decode_tokens_per_s']} tok/s "
                       f"decode ({rows[1]['prompt']}-token prompt + {rows[1]['decode_steps']} steps)",
                rows=rows)


def qpack3_cpu_decode(path3, threads):
    """the reference Container's QPACK3 decode (container.cpp:94-121: one task per coded blob or 16 MiB chunk, a pool of
    threads) with the reference codec compiled from its sources (oracle/_ref): returns (seconds, raw bytes)"""
    import ctypes as C
    import struct
    from concurrent.futures import ThreadPoolExecutor
    import oracle
    L = oracle.rlib()
    buf = np.fromfile(path3, np.uint8)
    n = struct.unpack("<I", buf[8:12].tobytes())[0]
    toc = {}
    for i in range(n):
        b = 16 + 72 * i
        name = buf[b:b + 56].tobytes().rstrip(b"\0").decode()
        toc[name] = struct.unpack("<QQ", buf[b + 56:b + 72].tobytes())
    off, ln = toc["manifest.json"]
    enc = json.loads(buf[off:off + ln].tobytes())["encoded"]
    tasks = []   # (offset, length, raw)
    for name in enc:
        off, ln = toc[name]
        if buf[off] == 3:
            cr, nc = struct.unpack("<II", buf[off + 6:off + 14].tobytes())
            lens = np.frombuffer(buf[off + 14:off + 14 + 4 * nc].tobytes(), np.uint32)
            pos = off + 14 + 4 * nc
            for cl in lens:
                tasks.append((pos, int(cl), struct.unpack("<I", buf[pos + 2:pos + 6].tobytes())[0]))
                pos += int(cl)
        else:
            tasks.append((off, ln, struct.unpack("<I", buf[off + 2:off + 6].tobytes())[0]))
    outs = [np.empty(r + 16, np.uint8) for _, _, r in tasks]
    base = buf.ctypes.data

    def one(i):
        o, l, _ = tasks[i]
        if L.qpref_rans_decode(C.c_void_p(base + o), l, outs[i].ctypes.data_as(C.c_void_p)):
            raise RuntimeError(L.qpref_error().decode())
    t = time.perf_counter()
    with ThreadPoolExecutor(threads) as ex:
        list(ex.map(one, range(len(tasks))))
    return time.perf_counter() - t, sum(r for _, _, r in tasks)


def graph_timeline(path):
    """Summary of the per-launch lines QPH_GRAPH_STAMPS writes for the last replayed decode step: kernel name, earliest
    wave start and latest wave end in 100 MHz realtime ticks, in launch order."""
    rows = [l.split() for l in open(path) if l.strip()]
    names = [r[0] for r in rows]
    t = [(int(r[1]) / 100.0, int(r[2]) / 100.0) for r in rows]   # us
    span = t[-1][1] - t[0][0]
    per, gaps = {}, {}
    for i, (n, (b, e)) in enumerate(zip(names, t)):
        per.setdefault(n, []).append(e - b)
        if i + 1 < len(t):
            gaps.setdefault(n + "->" + names[i + 1], []).append(t[i + 1][0] - e)
    busy = sum(e - b for b, e in t)
    mean = lambda v: round(sum(v) / len(v), 2)
    return {"launches": len(rows), "span_us": round(span, 1), "kernel_us": round(busy, 1),
            "kernel_frac": round(busy / span, 4),
            "kernel_mean_us": {n: mean(v) for n, v in per.items()},
            "gap_mean_us": {n: mean(v) for n, v in gaps.items()},
            "note": "last timed step, replayed from its HIP graph: first wave start to last wave end of every stamped "
                    "launch (the matvecs and k_attn_wo; embedding and argmax finish are not stamped)"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed greedy decode tokens")
    ap.add_argument("--warmup", type=int, default=8, help="untimed greedy decode tokens before the timed ones")
    ap.add_argument("--config", default="c3", help="synthetic shape (qpack_amd.CONFIGS key)")
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--prefill-tokens", type=int, default=2048)
    ap.add_argument("--kernel-iters", type=int, default=100)
    ap.add_argument("--model", help="use this .qpack instead of synthesising one")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-qpack3", action="store_true", help="skip the QPACK3 (rANS-coded) load leg")
    ap.add_argument("--configs", default="c1,c2,c5",
                    help="other benchmark configurations whose decode rate is added to the line ('' for none)")
    ap.add_argument("--profile", action="store_true",
                    help="launch kernels one by one (no HIP graphs) so a profiler sees every dispatch, and run a "
                         "calibration copy of known size for the byte counters")
    ap.add_argument("--dominant", choices=sorted(DOMINANT), default="norm",
                    help="which gate / up kernel --pmc-summary reads: 'norm' (PRO_NORM, what the token loop runs) or "
                         "'sum' (PRO_NORM_SUM, run only under QPH_AWO_SUM=0)")
    ap.add_argument("--graph-timeline", metavar="FILE",
                    help="capture the decode graphs with per-launch realtime stamps (QPH_GRAPH_STAMPS) and add the "
                         "last timed step's launches - per-kernel in-kernel time and the gaps between launches - to "
                         "the line as graph_timeline (the raw per-launch lines go to FILE)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the dominant kernel's per-launch HBM traffic from two rocprofv3 --pmc runs "
                         "(FETCH_SIZE, WRITE_SIZE) of --profile, scaled by the calibration copy; no GPU work")
    a = ap.parse_args()
    if a.pmc_summary:
        scale_note = []
        total = 0.0
        for path, ctr in zip(a.pmc_summary, ("FETCH_SIZE", "WRITE_SIZE")):
            k, cp, nk, ncp = pmc_summary(path, DOMINANT[a.dominant][0])[ctr]
            f = (COPY_BYTES / 1024) / cp            # counter reads KiB; the copy moves COPY_BYTES each way
            total += k * 1024 * f
            scale_note.append(f"{ctr}: kernel {k:.1f} KiB/dispatch over {nk} dispatches; copy {cp:.1f} KiB/dispatch "
                              f"over {ncp} (expected {COPY_BYTES // 1024}) -> scale {f:.4f} -> {k * 1024 * f:.0f} B")
        print("\n".join(scale_note))
        print(f"traffic_bytes: {total:.0f}")
        return
    if a.profile:
        os.environ["QPH_NO_GRAPH"] = "1"
    if a.graph_timeline:
        if a.profile:
            print("bench.py: --graph-timeline needs the graphs (drop --profile)", file=sys.stderr)
            sys.exit(2)
        os.environ["QPH_GRAPH_STAMPS"] = a.graph_timeline
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {a.gpus}); the multi-GPU sharding plan is "
              "documented as a design, not built", file=sys.stderr)
        sys.exit(2)

    import qpack_amd as qa
    if qa.device_count() < 1:
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    shape = qa.CONFIGS[a.config]
    tmpdir = None
    path = a.model
    if not path:
        tmpdir = tempfile.mkdtemp(prefix="qpack_bench_")
        path = os.path.join(tmpdir, f"{a.config}.qpack")
        t = time.time()
        qa.write_synthetic(a.config, path, seed=a.seed, threads=min(16, os.cpu_count() or 8))
        log(f"synthesised {a.config} ({os.path.getsize(path) / 2**30:.2f} GiB) in {time.time() - t:.1f}s")
    ctx = max(a.prompt + a.warmup + a.steps + 8, (0 if a.no_prefill else a.prefill_tokens) + 8)
    t = time.time()
    m = qa.HipLlama.load(path, max_ctx=ctx)
    log(f"loaded into HBM in {time.time() - t:.1f}s (max_ctx {ctx})")

    rng = np.random.default_rng(a.seed)
    prompt = rng.integers(0, shape.vocab, a.prompt).astype(np.int32)
    lg = m.prefill(prompt, 1)
    tok = int(np.argmax(lg))
    if a.warmup:
        tok = int(m.greedy_run(tok, a.warmup)[-1])
    T0 = m.pos()
    t0 = time.perf_counter()
    ms = m.time_greedy(tok, a.steps)
    wall = time.perf_counter() - t0
    T1 = m.pos()
    tok_s = a.steps / (ms / 1e3)
    mean_T = (T0 + 1 + T1) / 2
    sb = step_bytes(file_weight_bytes(path), shape, mean_T)
    step_gbs = sb / (ms / 1e3 / a.steps) / 1e9
    log(f"decode: {a.steps} tokens in {ms:.2f} ms (HIP events), wall {wall * 1e3:.2f} ms -> {tok_s:.1f} tok/s, "
        f"{step_gbs:.0f} GB/s algorithmic ({100 * step_gbs / HBM_PEAK_GBS:.1f}% of peak)")
    timeline = None
    if a.graph_timeline:   # written by the timed time_greedy; later models load without the hook
        timeline = graph_timeline(a.graph_timeline)
        os.environ.pop("QPH_GRAPH_STAMPS", None)
        log(f"graph timeline: {json.dumps(timeline)}")

    if a.profile:
        calibration_copy()
    dom = "sum" if os.environ.get("QPH_AWO_SUM") == "0" else "norm"
    try:
        kms, kbytes = m.time_kernel(DOMINANT[dom][1], a.kernel_iters)
    except RuntimeError:   # a model the fused attention + wo kernel does not take
        dom = "norm"
        kms, kbytes = m.time_kernel(DOMINANT[dom][1], a.kernel_iters)
    k_gbs = kbytes / (kms / 1e3) / 1e9
    log(f"dominant kernel ({DOMINANT[dom][0]}): {kms * 1e3:.2f} us, {kbytes / 1e6:.1f} MB -> {k_gbs:.0f} GB/s")
    others = {}
    plain = [(0, "gate_up_plain")] if dom == "sum" else []   # the same product without the partials, for comparison
    for which, name in [(1, "down"), (2, "qkv"), (3, "wo"), (4, "head"), (5, "attention")] + plain:
        ks, kb = m.time_kernel(which, a.kernel_iters)
        others[name] = dict(us=round(ks * 1e3, 2), mbytes=round(kb / 1e6, 3), gbs=round(kb / (ks / 1e3) / 1e9, 1))
        log(f"  {name}: {ks * 1e3:.2f} us, {kb / 1e6:.2f} MB -> {kb / (ks / 1e3) / 1e9:.0f} GB/s")
    if m.pos() <= 1024:   # the fused attention + wo kernel the token loop runs at these contexts (q8 wo shapes)
        try:
            ks, kb = m.time_kernel(6, a.kernel_iters)
            others["attn_wo"] = dict(us=round(ks * 1e3, 2), mbytes=round(kb / 1e6, 3), gbs=round(kb / (ks / 1e3) / 1e9, 1))
            log(f"  attn_wo (fused): {ks * 1e3:.2f} us, {kb / 1e6:.2f} MB -> {kb / (ks / 1e3) / 1e9:.0f} GB/s")
        except RuntimeError:
            pass

    prefill = None
    if not a.no_prefill:
        p2 = rng.integers(0, shape.vocab, a.prefill_tokens).astype(np.int32)
        m.reset()
        m.prefill(p2[:256], 1)          # warm-up: first launches of the prompt kernels
        m.reset()
        t = time.perf_counter()
        m.prefill(p2, 1)
        pt = time.perf_counter() - t
        # algorithmic integer ops of the projections (2 per weight x token) and fp ops of causal attention
        macs_tok = shape.layers * (shape.hidden * (shape.heads + 2 * shape.kv_heads) * shape.head_dim
                                   + shape.heads * shape.head_dim * shape.hidden + 3 * shape.hidden * shape.ffn)
        gemm_ops = 2.0 * a.prefill_tokens * macs_tok
        T = a.prefill_tokens
        attn_flops = 2.0 * 2 * shape.layers * shape.heads * shape.head_dim * (T * (T + 1) / 2)
        prefill = dict(tokens=T, seconds=round(pt, 4), tokens_per_s=round(T / pt, 1),
                       int8_tops_algorithmic=round(gemm_ops / pt / 1e12, 1),
                       mfma_int8_frac_of_peak=round(2 * gemm_ops / pt / 5.0e15, 4),
                       attention_tflops=round(attn_flops / 1e12, 3),
                       path="int8 MFMA products over two activation planes (2 x the algorithmic ops executed), "
                            "f16 MFMA causal attention; whole-prompt wall time incl. last-token logits")
        log(f"prefill {T} tokens: {pt * 1e3:.1f} ms -> {T / pt:.0f} tok/s, {gemm_ops / pt / 1e12:.1f} algorithmic int8 TOP/s")
    m.close()

    others_cfg = {}
    for name in [c for c in a.configs.split(",") if c]:
        t = time.time()
        others_cfg[name] = other_config(name, a.seed)
        log(f"{name}: {others_cfg[name]['tokens_per_s']} tok/s, {others_cfg[name]['hbm_pct_of_peak']}% of HBM peak "
            f"({time.time() - t:.1f}s)")

    qpack3 = None
    if not a.no_qpack3:
        # the same weights rANS-coded (QPACK3, as qpack-pack writes them), loaded with the decode on the GPU
        path3 = path + ".qpack3"
        t = time.time()
        ncoded = qa.pack(path, path3, min(16, os.cpu_count() or 8))
        log(f"packed to QPACK3 ({ncoded} coded blobs, {os.path.getsize(path3) / 2**30:.2f} GiB) in {time.time() - t:.1f}s")
        t = time.perf_counter()
        m3 = qa.HipLlama.load(path3, max_ctx=64)
        load3 = time.perf_counter() - t
        st = m3.load_stats()
        m3.close()
        t = time.perf_counter()
        m2 = qa.HipLlama.load(path, max_ctx=64)
        load2 = time.perf_counter() - t
        m2.close()
        qpack3 = dict(planes=st["planes"], coded_bytes=st["coded_bytes"], raw_bytes=st["raw_bytes"],
                      decode_ms=round(st["decode_ms"], 2), upload_ms=round(st["upload_ms"], 2),
                      upload_decode_ms=round(st["total_ms"], 2), rounds=st["rounds"],
                      decode_gbs=round(st["raw_bytes"] / (st["decode_ms"] / 1e3) / 1e9, 2),
                      load_s=round(load3, 3), qpack2_load_s=round(load2, 3),
                      kernel="k_rans_decode: one wave per coded plane (16 MiB chunks); latency-bound per plane; one "
                             "launch per upload round, the decode under the upload (decode_ms: first launch to last)",
                      cpu_baseline=None)
        log(f"QPACK3 load: {load3:.2f}s (QPACK2 {load2:.2f}s); upload {st['upload_ms']:.1f} ms in {st['rounds']} rounds "
            f"under the decode {st['decode_ms']:.1f} ms (both {st['total_ms']:.1f} ms) for {st['raw_bytes'] / 1e9:.2f} GB "
            f"raw over {st['planes']} planes -> {qpack3['decode_gbs']} GB/s")
        if not a.no_cpu_baseline:
            import oracle
            if oracle.ref_available():
                thr = min(16, os.cpu_count() or 1)
                sec, raw = qpack3_cpu_decode(path3, thr)
                qpack3["cpu_baseline"] = {"value": round(raw / sec / 1e9, 3), "unit": "GB/s raw", "cores": thr,
                                          "kind": "reference",
                                          "sample": f"every coded blob of this file ({raw / 1e9:.2f} GB raw), decoded as the "
                                                    f"reference Container does (one task per blob / 16 MiB chunk, {thr} threads)"}
                log(f"QPACK3 cpu baseline: {raw / sec / 1e9:.2f} GB/s on {thr} threads ({sec:.2f}s)")
        os.remove(path3)

    cpu = None
    if not a.no_cpu_baseline:
        if os.path.exists(REF_BENCH):
            t = time.time()
            cpu = cpu_baseline(path, min(16, os.cpu_count() or 1))
            log(f"cpu baseline: {cpu['value']} tok/s on {cpu['cores']} threads; rows {cpu['rows']} ({time.time() - t:.1f}s)")
        else:
            log("cpu baseline skipped: qpack_amd/integration/_build/qpack-bench is not built")
    if tmpdir:
        os.remove(path)
        os.rmdir(tmpdir)

    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tokens/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms / a.steps, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 weights x int16 activations -> int32 (fp32 epilogue, fp16 KV)",
        "data": f"synthetic: seeded N(0,0.02) random-init weights quantised to {quant_name(shape)} (seed {a.seed}), uniform "
                "random prompt ids",
        "config": {"workload": f"{a.config}: {shape.layers}-layer hidden-{shape.hidden} {quant_name(shape)} batch-1 decode, {a.prompt}-token prompt + {a.warmup} warm-up + "
                               f"{a.steps} timed greedy tokens, fp16 KV (context {T0}..{T1})",
                   "decode_tokens": a.steps, "prompt_tokens": a.prompt, "parallelism": "single GPU"},
        "hbm_pct_of_peak": round(100 * step_gbs / HBM_PEAK_GBS, 2),
        "step_roofline": {"bound": "hbm", "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(step_gbs / HBM_PEAK_GBS, 4), "bytes_per_token": round(sb)},
        "roofline": {"bound": "hbm", "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(k_gbs / HBM_PEAK_GBS, 4), "traffic": read_traffic(DOMINANT[dom][2]),
                     "kernel": DOMINANT[dom][3],
                     "bytes_per_launch": round(kbytes), "us_per_launch": round(kms * 1e3, 2)},
        "kernels": others,
        "prefill": prefill,
        "other_configs": others_cfg,
        "qpack3_load": qpack3,
        "cpu_baseline": cpu,
    }
    if timeline:
        out["graph_timeline"] = timeline
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
