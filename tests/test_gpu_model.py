"""GPU parity of the whole token loop (qp::Model surface over the C ABI) against the oracle on small seeded models.

Bar (the parity contract of this path's default order): logits within max-abs 1e-2 and relative 1e-3 of the reference,
identical greedy streams (up to a reference near-tie where a file's stream meets one: assert_greedy_agrees).  The
reference-order mode is checked bit for bit in test_gpu_golden.py.
"""
import os

import numpy as np
import pytest

import oracle as O
import qpack_amd as qa

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-2, 1e-3


def close(a, b):
    err = np.abs(a - b)
    return float(err.max()), bool(np.all(err <= np.maximum(ATOL, RTOL * np.abs(b))))


def assert_greedy_agrees(gpu, orc, tok, n, err):
    """the device greedy chain (gpu.greedy_run) against the oracle's greedy steps: identical tokens up to the first
    oracle step whose top-2 gap is below tie = 20 x the measured logit error - the default order's contract (a float
    order of its own, within the tolerance; the reference-order mode is the bit-exact one), as in test_gpu_golden"""
    g = gpu.greedy_run(tok, n)
    tie = max(20 * err, 1e-5)
    for i in range(n):
        lo = orc.step(tok, 1)
        want = int(np.argmax(lo))
        if int(g[i]) != want:
            top = np.sort(lo)[-2:]
            gap = float(top[1] - top[0])
            assert gap < tie, f"greedy step {i}: {int(g[i])} vs the oracle's {want}, its top-2 gap {gap:.3g} >= {tie:.3g}"
            print(f"greedy agrees for {i}/{n} steps, then a near-tie (oracle gap {gap:.3g} < {tie:.3g})", flush=True)
            return
        tok = want


@pytest.mark.parametrize("cfg", ["mini", "mini128", "mini_q4", "mini_q4m", "mini_q1", "mini_q1m", "mini_q4mb", "mini_q4h",
                                 "mini_odd", "mini_odd_q4", "mini_r7", "mini_r7h"])
def test_decode_and_greedy_match_oracle(cfg, synth):
    path = synth(cfg)
    gpu = qa.HipLlama.load(path, max_ctx=256)
    orc = O.Oracle(path, max_ctx=256)
    rng = np.random.default_rng(3)
    toks = rng.integers(0, gpu.vocab(), 70).astype(np.int32)
    print(f"{cfg}: prefill 70", flush=True)
    lg, lo = gpu.prefill(toks, 1), orc.prefill(toks, 1)
    err, ok = close(lg, lo)
    assert ok, f"prefill logits max|d| {err}"
    for t in rng.integers(0, gpu.vocab(), 6):
        err, ok = close(gpu.step(int(t), 1), orc.step(int(t), 1))
        assert ok, f"step logits max|d| {err}"
    g, o = gpu.greedy_run(int(np.argmax(lg)), 48), orc.greedy_run(int(np.argmax(lo)), 48)
    np.testing.assert_array_equal(g, o)
    assert gpu.pos() == orc.pos() == 70 + 6 + 48
    gpu.close(); orc.close()


def test_want_hidden_and_state_only(synth):
    path = synth("mini")
    gpu = qa.HipLlama.load(path, max_ctx=64)
    orc = O.Oracle(path, max_ctx=64)
    for t in (1, 2, 3):
        assert gpu.step(t, 0) is None
        orc.step(t, 0)
    err, ok = close(gpu.step(4, 2), orc.step(4, 2))
    assert ok, err
    assert gpu.pos() == 4


def test_snapshot_restore_rewind(synth):
    path = synth("mini128")
    gpu = qa.HipLlama.load(path, max_ctx=128)
    toks = np.arange(1, 20, dtype=np.int32)
    gpu.prefill(toks, 0)
    snap = gpu.snapshot()
    assert len(snap) == 4 + 2 * 2 * 19 * 128 * 2
    a = gpu.step(7, 1)
    gpu2 = qa.HipLlama.load(path, max_ctx=128)
    gpu2.restore(snap)
    assert gpu2.pos() == 19
    np.testing.assert_array_equal(gpu2.step(7, 1), a)
    assert gpu.rewind(19) and not gpu.rewind(50)
    np.testing.assert_array_equal(gpu.step(7, 1), a)
    c = gpu.checkpoint()
    gpu.step(8, 0)
    gpu.rollback(c)
    assert gpu.pos() == 20


@pytest.mark.parametrize("cfg,path,P", [("mini128", "fused", 45), ("mini128", "single", 45), ("mini128", "splits", 45),
                                        ("mini", "fused", 45), ("mini", "splits", 45), ("mini_r7", "fused", 45),
                                        ("mini128", "fused", 560), ("mini", "fused", 560)])
def test_stale_nan_rows_past_context(cfg, path, P, synth, monkeypatch):
    """cache rows past the context hold whatever a longer sequence left there - NaN here (a restored snapshot 19
    positions longer, then a rewind).  The decode attention loads whole 32-position blocks of K and V; the rows past
    the context (or past a split's end) must not reach the output: their scores are -inf and their V rows are zeroed
    in LDS (0 x NaN would be NaN).  The logits of every step through that region equal a clean cache's bit for bit, on
    the fused attention + wo kernel, the one-split attention kernel and forced small splits (a partial block at every
    split's end); at 560 positions the fused kernel's waves run three blocks each in its block loop"""
    if path != "fused":
        monkeypatch.setenv("QPH_AWO_MAX", "0")
    if path == "splits":
        monkeypatch.setenv("QPH_ATTN_SINGLE", "16")
        monkeypatch.setenv("QPH_ATTN_SPLIT_POS", "16")
    model = synth(cfg)
    shape = qa.CONFIGS[cfg]
    kvd = shape.kv_heads * shape.head_dim
    clean = qa.HipLlama.load(model, max_ctx=P + 80)
    dirty = qa.HipLlama.load(model, max_ctx=P + 80)
    rng = np.random.default_rng(5)
    extra = 19
    clean.prefill(rng.integers(0, clean.vocab(), P).astype(np.int32), 0)
    pos, k, v = split_snapshot(clean.snapshot(), shape.layers, kvd)
    assert pos == P
    nan = np.full((shape.layers, extra, kvd), np.nan, np.float16)
    body = np.stack([np.concatenate([k, nan], 1), np.concatenate([v, nan], 1)], 1)   # [layers][K, V][rows][kvd]
    dirty.restore(np.int32(P + extra).tobytes() + body.tobytes())
    assert dirty.rewind(P) and dirty.pos() == P
    print(f"{cfg} {path}: NaN rows {P}..{P + extra - 1}, steps {P}..{P + 24}", flush=True)
    for t in rng.integers(0, clean.vocab(), 25):
        a, b = clean.step(int(t), 1), dirty.step(int(t), 1)
        assert np.isfinite(b).all(), f"non-finite logits at position {dirty.pos() - 1}"
        np.testing.assert_array_equal(b, a)
    clean.close(); dirty.close()


def test_errors_are_reported(synth):
    path = synth("mini")
    gpu = qa.HipLlama.load(path, max_ctx=8)
    with pytest.raises(qa.QphError, match="out of range"):
        gpu.step(10**6, 1)
    gpu.prefill(np.arange(8, dtype=np.int32), 0)
    with pytest.raises(qa.QphError, match="context window full"):
        gpu.step(1, 1)
    assert len(gpu.greedy_run(1, 4)) == 0
    with pytest.raises(qa.QphError):
        qa.HipLlama.load("/nonexistent.qpack")


def split_snapshot(snap, layers, kvd):
    """the reference snapshot layout (model_llama.cpp:55-63): int32 pos, then per layer K rows then V rows (fp16)"""
    pos = int(np.frombuffer(snap[:4], np.int32)[0])
    body = np.frombuffer(snap[4:], np.float16).reshape(layers, 2, pos, kvd)
    return pos, body[:, 0], body[:, 1]


@pytest.mark.parametrize("cfg,chunk", [("mini", 48), ("mini128", 0), ("mini128", 37), ("mini_odd", 0), ("mini_odd_q4", 29)])
def test_batched_prefill(cfg, chunk, synth, monkeypatch):
    """the int8-MFMA prompt path: chunked (ragged last chunk), a second prompt continuing at p0 > 0; logits and every
    cache row against the oracle (within the tolerance / fp16 rounding), the greedy continuation identical, and the
    layer-0 cache rows bit-identical to the GPU's own decode-step path for q8 (exact products, same quantised
    activations, same RoPE and fp16 rounding; the decode path differs from the reference only by its RMSNorm summation
    order); for q4 within one fp16 rounding step (the prompt product's group sums run in another float order)"""
    if chunk:
        monkeypatch.setenv("QPH_PF_CHUNK", str(chunk))
    path = synth(cfg)
    gpu = qa.HipLlama.load(path, max_ctx=256)
    orc = O.Oracle(path, max_ctx=256)
    rng = np.random.default_rng(11)
    toks = rng.integers(0, gpu.vocab(), 150).astype(np.int32)
    prompts = ((0, 100), (100, 150))
    for a, b in prompts:
        print(f"{cfg} chunk {chunk}: prefill [{a}, {b})", flush=True)
        lg = gpu.prefill(toks[a:b], 1)
        for t in toks[a:b]:
            lo = orc.step(int(t), 1)
        err, ok = close(lg, lo)
        assert ok, f"prefill [{a}, {b}) logits max|d| {err}"
    shape = qa.CONFIGS[cfg]
    kvd = shape.kv_heads * shape.head_dim
    pos, kb, vb = split_snapshot(gpu.snapshot(), shape.layers, kvd)
    assert pos == 150
    ko, vo = orc.kv_cache()
    for a, b in ((kb, ko[:, :150].view(np.float16)), (vb, vo[:, :150].view(np.float16))):
        d = np.abs(a.astype(np.float32) - b.astype(np.float32))
        assert d.max() <= 1e-2 + 2e-3 * np.abs(b.astype(np.float32)).max(), float(d.max())
    g, o = gpu.greedy_run(int(np.argmax(lg)), 32), orc.greedy_run(int(np.argmax(lo)), 32)
    np.testing.assert_array_equal(g, o)
    gpu.reset()
    monkeypatch.setenv("QPH_PREFILL_STEPS", "1")
    for a, b in prompts:
        gpu.prefill(toks[a:b], 0)
    _, ks, vs = split_snapshot(gpu.snapshot(), shape.layers, kvd)
    for a, b in ((kb[0], ks[0]), (vb[0], vs[0])):
        if not shape.q4:
            np.testing.assert_array_equal(a.view(np.uint16), b.view(np.uint16))
        else:   # q4 products sum their groups in another float order than rows_q4: within one fp16 rounding step
            a32, b32 = a.astype(np.float32), b.astype(np.float32)
            assert np.all(np.abs(a32 - b32) <= np.abs(b32) * 2.0 ** -10 + 2.0 ** -24), float(np.abs(a32 - b32).max())
    gpu.close(); orc.close()


def test_batched_prefill_equals_step_path(synth, monkeypatch):
    """the batched prompt path and the decode-step path agree (logits within the tolerance, same greedy pick)"""
    path = synth("mini128")
    toks = np.random.default_rng(5).integers(0, 2048, 90).astype(np.int32)
    gpu = qa.HipLlama.load(path, max_ctx=128)
    lb = gpu.prefill(toks, 1)
    gpu.reset()
    monkeypatch.setenv("QPH_PREFILL_STEPS", "1")
    ls = gpu.prefill(toks, 1)
    gpu.close()
    err, ok = close(lb, ls)
    assert ok, err
    assert int(np.argmax(lb)) == int(np.argmax(ls))


@pytest.mark.parametrize("cfg", ["mini", "mini128", "mini_odd", "c1"])
def test_prefill_q8_kernels_agree(cfg, synth, monkeypatch):
    """the two q8 prompt-product kernels (16 x 16 and 32 x 32 MFMA tiles, forced with QPH_GEMM=2 / 1) carry out the
    same arithmetic: a 300-token prompt gives bit-identical logits and cache rows with either, the 32 x 32 kernel then
    running every product of the prompt (the q / k / v segments with bias, wo / down into the residual, the gate / up
    pair with SwiGLU and its quantised store); and so does the launcher's own choice for 8 CUs, which splits the
    q / k / v launch over both kernels, and the prompt with no fusions (QPH_PF_UNFUSED: q rotated by k_pf_rope, the
    attention and SwiGLU outputs quantised by k_pf_quant)"""
    path = synth(cfg)
    toks = np.random.default_rng(17).integers(0, qa.CONFIGS[cfg].vocab, 300).astype(np.int32)
    out = []
    for k in ("2", "1", "auto8", "unfused"):
        if k == "auto8":   # the launcher's own choice for 8 CUs: q / k / v split over both kernels
            monkeypatch.delenv("QPH_GEMM")
            monkeypatch.setenv("QPH_GEMM_CUS", "8")
        elif k == "unfused":   # q's RoPE and the output quantisations as launches of their own
            monkeypatch.setenv("QPH_PF_UNFUSED", "7")
        else:
            monkeypatch.setenv("QPH_GEMM", k)
        print(f"{cfg}: 300-token prompt, QPH_GEMM={k}", flush=True)
        gpu = qa.HipLlama.load(path, max_ctx=320)
        lg = gpu.prefill(toks, 1)
        out.append((lg, gpu.snapshot()))
        gpu.close()
    for o in out[1:]:
        np.testing.assert_array_equal(out[0][0], o[0])
        assert out[0][1] == o[1], "cache rows differ between the kernels"


def kv_snapshot(k, v):
    """a snapshot in the reference layout (model_llama.cpp:55-63) from per-layer fp16 K / V rows [L][pos][kvd]"""
    pos = k.shape[1]
    parts = [np.int32(pos).tobytes()]
    for layer in range(k.shape[0]):
        parts += [np.ascontiguousarray(k[layer]).tobytes(), np.ascontiguousarray(v[layer]).tobytes()]
    return b"".join(parts)


@pytest.mark.parametrize("cfg,T", [("mini_q4m", 3000), ("mini128", 2500), ("mini_r7", 1500), ("mini_r7h", 1200),
                                   ("mini", 700), ("mini128", 400)])
def test_long_context_restore(cfg, T, synth):
    """decode at a long restored context (N(0,1) fp16 keys / values, as the C5 workload fills its 16K cache): many
    context splits per kv group and their merge; logits against the oracle holding the same cache, then greedy"""
    path = synth(cfg)
    shape = qa.CONFIGS[cfg]
    kvd = shape.kv_heads * shape.head_dim
    rng = np.random.default_rng(T)
    k = rng.standard_normal((shape.layers, T, kvd)).astype(np.float16)
    v = rng.standard_normal((shape.layers, T, kvd)).astype(np.float16)
    gpu = qa.HipLlama.load(path, max_ctx=T + 64)
    gpu.restore(kv_snapshot(k, v))
    assert gpu.pos() == T
    orc = O.Oracle(path, max_ctx=T + 64)
    ko, vo = orc.kv_cache()
    ko[:, :T] = k.view(np.uint16); vo[:, :T] = v.view(np.uint16)
    orc.set_pos(T)
    print(f"{cfg}: context {T}", flush=True)
    for t in (5, 17, 230):
        lg, lo = gpu.step(t, 1), orc.step(t, 1)
        err, ok = close(lg, lo)
        assert ok, f"step logits max|d| {err}"
    g, o = gpu.greedy_run(int(np.argmax(lg)), 16), orc.greedy_run(int(np.argmax(lo)), 16)
    np.testing.assert_array_equal(g, o)
    gpu.close(); orc.close()


@pytest.mark.parametrize("cfg,T", [("mini_r7", 1500), ("mini128", 2100), ("mini_q4m", 990)])
def test_attention_separate_merge(cfg, T, synth, monkeypatch):
    """long contexts (every step >= 16 splits per kv group) merge the splits in a launch of their own (k_attn_merge):
    the logits equal the in-kernel merge's (QPH_ATTN_MERGE_SEP=0) bit for bit - the same merge arithmetic - at every
    step and in graph-replayed greedy runs, and match the oracle; a run that starts below the threshold and crosses it
    (mini_q4m: 990 = 15 x 64 + 30 positions, the threshold 961) switches graphs on the way"""
    path = synth(cfg)
    shape = qa.CONFIGS[cfg]
    kvd = shape.kv_heads * shape.head_dim
    rng = np.random.default_rng(T + 1)
    T0 = T - 40 if cfg == "mini_q4m" else T
    k = rng.standard_normal((shape.layers, T0, kvd)).astype(np.float16)
    v = rng.standard_normal((shape.layers, T0, kvd)).astype(np.float16)
    snap = kv_snapshot(k, v)
    sep = qa.HipLlama.load(path, max_ctx=T + 96)
    monkeypatch.setenv("QPH_ATTN_MERGE_SEP", "0")
    ink = qa.HipLlama.load(path, max_ctx=T + 96)
    monkeypatch.delenv("QPH_ATTN_MERGE_SEP")
    orc = O.Oracle(path, max_ctx=T + 96)
    ko, vo = orc.kv_cache()
    ko[:, :T0] = k.view(np.uint16); vo[:, :T0] = v.view(np.uint16)
    orc.set_pos(T0)
    for m in (sep, ink):
        m.restore(snap)
    print(f"{cfg}: context {T0}, separate against in-kernel merge", flush=True)
    for i in range(50):
        t = int(rng.integers(0, shape.vocab))
        a, b, c = sep.step(t, 1), ink.step(t, 1), orc.step(t, 1)
        np.testing.assert_array_equal(a, b, err_msg=f"step at {sep.pos()}")
        err, ok = close(a, c)
        assert ok, f"step at {sep.pos()}: logits max|d| {err}"
    p0 = sep.pos()
    tok = int(np.argmax(a))
    ga = sep.greedy_run(tok, 24)
    gb = ink.greedy_run(tok, 24)
    np.testing.assert_array_equal(ga, gb)
    np.testing.assert_array_equal(ga, orc.greedy_run(tok, 24))
    assert sep.rewind(p0) and ink.rewind(p0)
    np.testing.assert_array_equal(sep.greedy_run(tok, 24), ga)
    sep.close(); ink.close(); orc.close()


REF_QUANT = os.path.join(os.path.dirname(O.REF_LIB), "qpack-quantize")


@pytest.mark.skipif(not os.path.exists(REF_QUANT), reason="oracle/_ref/qpack-quantize not built")
@pytest.mark.parametrize("src,args", [("mini128", ["--type", "q1"]), ("mini", ["--type", "q1", "--q1-attn", "q4"]),
                                      ("mini128", ["--type", "q4", "--q4-head"]), ("mini_q4m", ["--type", "q4m"])])
def test_files_of_the_reference_quantiser(src, args, synth, tmp_path):
    """files written by the reference's own qpack-quantize (q1 MLP, q1 with q4 attention, q4 head, q4m policy) from a
    synthetic q8 / q4m model: logits within the bar and the greedy stream against the oracle's up to a near-tie"""
    import subprocess
    path = str(tmp_path / "rq.qpack")
    subprocess.run([REF_QUANT, synth(src), path] + args, check=True, capture_output=True)
    gpu = qa.HipLlama.load(path, max_ctx=160)
    orc = O.Oracle(path, max_ctx=160)
    rng = np.random.default_rng(5)
    toks = rng.integers(0, gpu.vocab(), 40).astype(np.int32)
    print(f"reference-quantised {src} {args}", flush=True)
    lg, lo = gpu.prefill(toks, 1), orc.prefill(toks, 1)
    err, ok = close(lg, lo)
    assert ok, f"prefill logits max|d| {err}"
    assert int(np.argmax(lg)) == int(np.argmax(lo))
    assert_greedy_agrees(gpu, orc, int(np.argmax(lo)), 32, err)
    gpu.close(); orc.close()


def test_attention_merge_timeout_is_an_error(synth, monkeypatch):
    """the decode attention's failure path, forced from the host (QPH_ATTN_FORCE_LATE, read at load: every merger
    that would wait gives up at once, as when its bounded wait runs out): it writes NaN and sets the status word; the
    call raises instead of returning those outputs, the split counters are cleared, the position returns to the last
    clean wait, and every kernel still runs to completion (a fresh model
    at the same context decodes normally afterwards)"""
    cfg, T = "mini_r7", 1500   # 24 splits per kv group, 7 heads per group: the parallel merge with waiting mergers
    path = synth(cfg)
    shape = qa.CONFIGS[cfg]
    kvd = shape.kv_heads * shape.head_dim
    rng = np.random.default_rng(11)
    k = rng.standard_normal((shape.layers, T, kvd)).astype(np.float16)
    v = rng.standard_normal((shape.layers, T, kvd)).astype(np.float16)
    snap = kv_snapshot(k, v)
    monkeypatch.setenv("QPH_ATTN_FORCE_LATE", "1")
    monkeypatch.setenv("QPH_ATTN_MERGE_SEP", "0")   # the in-kernel merge (the default merges long contexts in a launch)
    bad = qa.HipLlama.load(path, max_ctx=T + 64)
    monkeypatch.delenv("QPH_ATTN_FORCE_LATE")
    monkeypatch.delenv("QPH_ATTN_MERGE_SEP")
    bad.restore(snap)
    with pytest.raises(qa.QphError, match="timed out"):
        bad.step(5, 1)
    assert bad.pos() == T, "a failed step must leave the position where the call found it"
    with pytest.raises(qa.QphError, match="timed out"):
        bad.greedy_run(5, 4)
    assert bad.pos() == T
    # state-only steps run ahead of any wait: the failure surfaces at the next wait, and the position goes back to
    # the last clean check (here the restore), not just one step
    bad.step(5, 0); bad.step(6, 0)
    with pytest.raises(qa.QphError, match="timed out"):
        bad.step(7, 1)
    assert bad.pos() == T
    bad.close()
    good = qa.HipLlama.load(path, max_ctx=T + 64)
    good.restore(snap)
    orc = O.Oracle(path, max_ctx=T + 64)
    ko, vo = orc.kv_cache()
    ko[:, :T] = k.view(np.uint16); vo[:, :T] = v.view(np.uint16)
    orc.set_pos(T)
    err, ok = close(good.step(5, 1), orc.step(5, 1))
    assert ok, err
    good.close(); orc.close()


def test_graph_replays_with_device_logits(synth):
    """many back-to-back graph replays whose logits stay on the device (step_topk: want = 3, no host wait inside the
    step), past two turns of the 256-slot control ring, each checked against step(tok, 1) on a twin model"""
    path = synth("c1") if os.environ.get("QPH_TEST_C1") else synth("mini")
    a = qa.HipLlama.load(path, max_ctx=700)
    b = qa.HipLlama.load(path, max_ctx=700)
    toks = np.arange(3, 35, dtype=np.int32) % a.vocab()
    a.prefill(toks, 0); b.prefill(toks, 0)
    print("step_topk x 600", flush=True)
    for i in range(600):
        t = (100 + 7 * i) % a.vocab()
        M = 40 if i % 2 else 512
        idx, val = a.step_topk(t, M)
        lg = b.step(t, 1)
        order = np.lexsort((np.arange(len(lg)), -lg.astype(np.float64)))[:M]
        np.testing.assert_array_equal(idx, order)
        np.testing.assert_array_equal(val, lg[order])
    assert a.pos() == b.pos() == 32 + 600
    a.close(); b.close()


@pytest.mark.parametrize("cfg", ["mini", "mini128", "mini_odd", "mini_r7h", "mini_r7"])
def test_fused_attention_wo(cfg, synth, monkeypatch):
    """decode attention fused with the wo product and residual (contexts up to QPH_AWO_MAX positions) against the
    oracle and against the split attention + wo matvec launches, across the threshold (fused up to 100 positions,
    split beyond), then greedy chains of both against the oracle's.  k_attn_wo (per kv group, partials summed by
    gate / up) for groups of whole 128-column blocks; k_attn_wo_rows (every group, whole rows) for mini_r7's groups of
    7 heads of 64, whose logits must equal the split launches' bit for bit.  k_attn_wo's group partials are added to the
    residual stream by each row chunk's last workgroup (default) or by the gate / up prologue (QPH_AWO_SUM=0): both
    forms are checked"""
    path = synth(cfg)
    rows = cfg == "mini_r7"   # 7 heads of 64 per group: k_attn_wo_rows, bit-identical to the split launches
    monkeypatch.setenv("QPH_AWO_MAX", "100")
    models = [qa.HipLlama.load(path, max_ctx=192)]
    if not rows:
        monkeypatch.setenv("QPH_AWO_SUM", "0")
        models.append(qa.HipLlama.load(path, max_ctx=192))
        monkeypatch.delenv("QPH_AWO_SUM")
    monkeypatch.setenv("QPH_AWO_MAX", "0")
    split = qa.HipLlama.load(path, max_ctx=192)
    monkeypatch.delenv("QPH_AWO_MAX")
    orc = O.Oracle(path, max_ctx=192)
    rng = np.random.default_rng(21)
    toks = rng.integers(0, split.vocab(), 60).astype(np.int32)
    print(f"{cfg}: fused attention + wo ({len(models)} forms), prompt 60, steps to 110", flush=True)
    for m in models + [split]:
        m.prefill(toks, 0)
    lo = orc.prefill(toks, 1)
    for t in rng.integers(0, split.vocab(), 50):
        b, c = split.step(int(t), 1), orc.step(int(t), 1)
        err, ok = close(b, c)
        assert ok, f"split step at {split.pos()}: logits max|d| {err} against the oracle"
        for i, m in enumerate(models):
            a = m.step(int(t), 1)
            if rows:
                np.testing.assert_array_equal(a, b)
            err, ok = close(a, c)
            assert ok, f"fused form {i} step at {m.pos()}: logits max|d| {err} against the oracle"
        lo = c
    # greedy from position 70 (fused for the first 30 steps, then split)
    for m in models + [split]:
        assert m.rewind(70)
    orc.set_pos(70)
    tok = int(np.argmax(lo))
    o = orc.greedy_run(tok, 40)
    for m in models + [split]:
        np.testing.assert_array_equal(m.greedy_run(tok, 40), o)
        m.close()
    orc.close()


@pytest.mark.gpu
def test_graph_timeline_hook(synth, monkeypatch, tmp_path):
    """QPH_GRAPH_STAMPS: the graphs are captured with per-launch realtime stamps and time_greedy writes the last
    replayed step's launches (4 per layer and the head, in launch order, each ending after it starts and starting
    no earlier than the previous one started), without changing the tokens."""
    path = synth("mini")
    ref = qa.HipLlama.load(path, max_ctx=128)
    want = ref.greedy_run(5, 12)
    out = tmp_path / "tl.txt"
    monkeypatch.setenv("QPH_GRAPH_STAMPS", str(out))
    m = qa.HipLlama.load(path, max_ctx=128)
    m.time_greedy(5, 12)
    rows = [l.split() for l in out.read_text().splitlines()]
    names = [r[0] for r in rows]
    assert names == ["qkv", "attn_wo", "gate_up", "down"] * m.config.layers + ["head"], names
    t = [(int(r[1]), int(r[2])) for r in rows]
    assert all(b < e for b, e in t)
    assert all(t[i + 1][0] >= t[i][0] for i in range(len(t) - 1))
    m.rewind(0); ref.rewind(0)
    assert list(m.greedy_run(5, 12)) == list(want)
