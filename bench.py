#!/usr/bin/env python3
"""Batched-decode throughput of the MI355X backend on the reference's headline
workload: a random-init Qwen3.5-0.8B-shaped hybrid model (24 layers, 3
GatedDeltaNet : 1 gated attention, Q4-G32-DOT4 H128 weights), 16 requests with
512-token random prompts, greedy decode.

One step = one decode forward of the 16-row batch through CpuEngine's
advance_batch equivalent (q35_engine_advance_batch): host scheduling, one
metadata upload, the captured step graph, the fused greedy head and the token
read-back. Throughput counts decode forwards x rows / seconds, the reference's
definition (src/cpu_engine_bench_main.cpp:301).

After the timed region, a profiled region of the same decode (eager launches,
HIP events on the runtime's stream around every kernel) gives per-kernel-class
durations and the roofline of the dominant kernel. The reference CPU engine,
built from the reference sources into oracle/_ref, is timed on a bounded sample
of the same workload as the baseline.

Prints one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POP/s
METRIC = "decode tokens/s at B=16 (0.8B random-init, 1 GPU); Q4 GEMV % peak HBM BW"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")

# the 0.8B text config the reference's ProfileLoader reads (profile_loader.cpp:320-420)
CONFIG_08B = {
    "_name_or_path": "Qwen/Qwen3.5-0.8B", "model_type": "qwen3_5",
    "text_config": {
        "model_type": "qwen3_5_text", "num_hidden_layers": 24, "hidden_size": 1024,
        "intermediate_size": 3584, "num_attention_heads": 8, "num_key_value_heads": 2, "head_dim": 256,
        "vocab_size": 248320, "max_position_embeddings": 32768, "rms_norm_eps": 1e-06,
        "tie_word_embeddings": True, "full_attention_interval": 4, "linear_conv_kernel_dim": 4,
        "linear_num_key_heads": 16, "linear_num_value_heads": 16, "linear_key_head_dim": 128,
        "linear_value_head_dim": 128,
        "rope_parameters": {"rope_theta": 10000000.0, "partial_rotary_factor": 0.25}}}


# the 4B text config (text_architecture qwen35_4b, profile_loader.cpp:439-462)
CONFIG_4B = {
    "_name_or_path": "Qwen/Qwen3.5-4B", "model_type": "qwen3_5",
    "text_config": {
        "model_type": "qwen3_5_text", "num_hidden_layers": 32, "hidden_size": 2560,
        "intermediate_size": 9216, "num_attention_heads": 16, "num_key_value_heads": 4, "head_dim": 256,
        "vocab_size": 248320, "max_position_embeddings": 32768, "rms_norm_eps": 1e-06,
        "tie_word_embeddings": True, "full_attention_interval": 4, "linear_conv_kernel_dim": 4,
        "linear_num_key_heads": 16, "linear_num_value_heads": 32, "linear_key_head_dim": 128,
        "linear_value_head_dim": 128,
        "rope_parameters": {"rope_theta": 10000000.0, "partial_rotary_factor": 0.25}}}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def prepare_model_dir(q, seed, weight_std, encodings="q4"):
    """Writes the random-init artifact (and the reference's config.json) once per host;
    encodings "g16q8" selects the G16 tied head and the Q8_0 gate rows."""
    d, sched = q.model_dims(0)
    suffix = "" if encodings == "q4" else f"_{encodings}"
    path = os.path.join(tempfile.gettempdir(), f"q35_bench_0p8b_s{seed}{suffix}")
    os.makedirs(path, exist_ok=True)
    art = os.path.join(path, "model.q35h128")
    if not os.path.exists(art):
        t = time.time()
        alt = encodings != "q4"
        q.write_random_artifact(art + ".part", d, sched, seed=seed, weight_std=weight_std, head_g16=alt,
                                q8_gates=alt)
        os.replace(art + ".part", art)
        log(f"wrote random-init artifact {art} ({os.path.getsize(art) / 1e6:.1f} MB) in {time.time() - t:.1f}s")
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(CONFIG_08B, f)
    return d, sched, path, art


def host_cpus(threads):
    """The CPUs the baseline runs on: one logical CPU per physical core of the
    process's allowed set where the topology is readable (so `threads`
    workers land on distinct cores), then the CPU model and the counts."""
    allowed = sorted(os.sched_getaffinity(0))
    cores, seen = [], set()
    for c in allowed:
        try:
            with open(f"/sys/devices/system/cpu/cpu{c}/topology/core_id") as f:
                core = f.read().strip()
            with open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id") as f:
                pkg = f.read().strip()
        except OSError:
            core, pkg = str(c), "0"
        if (pkg, core) not in seen:
            seen.add((pkg, core))
            cores.append(c)
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    use = (cores + [c for c in allowed if c not in cores])[:threads]
    return use, model, len(allowed), len(cores)


def cpu_baseline(model_dir, artifact, batch, prompt_len, new_tokens, threads):
    """The reference CpuEngine (oracle/_ref, built from the reference sources)
    on the same workload as cpu_engine_bench_main.cpp:241-301: `batch`
    requests, `prompt_len`-token prompts, `new_tokens` greedy outputs (127
    decode forwards per request at the default 128), Q8_0Backend::auto_select;
    decode forwards x rows / decode seconds. The process is pinned to
    `threads` CPUs, one per physical core where possible."""
    from oracle import q35_oracle as orc  # the checker build, timed as the baseline only

    if not orc.ref_available():
        log("oracle/_ref not built: no CPU baseline")
        return None
    r = orc.ref()
    cpus, cpu_model, allowed, physical = host_cpus(threads)
    threads = len(cpus)
    before = os.sched_getaffinity(0)
    os.sched_setaffinity(0, cpus)
    isa = r.ref_backend_name(r.ref_backend_resolve(0)).decode()  # auto_select resolved on this host
    rng = np.random.default_rng(4242)
    prompts = rng.integers(0, CONFIG_08B["text_config"]["vocab_size"], size=(batch, prompt_len)).astype(np.int32)
    out = np.zeros((batch, new_tokens), np.int32)
    ms = ctypes.c_double()
    err = ctypes.create_string_buffer(512)
    t = time.time()
    try:
        rc = r.ref_engine_greedy(os.fsencode(model_dir), os.fsencode(artifact), threads, 0, prompts.ctypes.data,
                                 prompt_len, batch, new_tokens, 1.0, None, out.ctypes.data, None, None,
                                 ctypes.byref(ms), err, 512)
    finally:
        os.sched_setaffinity(0, before)
    if rc != 0:
        log(f"reference engine failed: {err.value.decode(errors='replace')}")
        return None
    forwards = new_tokens - 1  # the first output token comes out of prefill
    value = batch * forwards * 1000.0 / ms.value
    log(f"reference CPU engine: {value:.1f} tok/s decode on {threads} threads pinned to CPUs {cpus} "
        f"({cpu_model}, {isa}; {physical} physical cores / {allowed} CPUs allowed) ({time.time() - t:.1f}s wall)")
    return {"value": round(value, 2), "unit": "tokens/s", "cores": threads, "kind": "reference",
            "cpu_model": cpu_model, "isa": isa, "threads": threads, "pinned_cpus": cpus,
            "allowed_cpus": allowed, "physical_cores_allowed": physical,
            "sample": f"{batch} requests x {prompt_len}-token random prompts, {new_tokens} greedy tokens each; "
                      f"{forwards} decode forwards per request timed through CpuEngine::advance_batch on the "
                      f"same random-init 0.8B artifact (cpu_engine_bench_main.cpp:241-301 workload), "
                      f"Q8_0Backend::auto_select -> {isa}, one thread per physical core of the box's CPU share"}


def projection_weights(d, sched):
    """Q4 weights of every layer's projections (not the head)."""
    H, I, hd = d.hidden, d.intermediate, d.head_dim
    q_dim, v_dim = d.lin_k_heads * d.lin_k_dim, d.lin_v_heads * d.lin_v_dim
    total = 0
    for linear in sched:
        if linear:
            total += (2 * q_dim + 2 * v_dim + 2 * d.lin_v_heads) * H + H * v_dim
        else:
            total += (2 * d.n_heads * hd + 2 * d.n_kv_heads * hd) * H + H * d.n_heads * hd
        total += 2 * I * H + H * I
    return total


def mfma_roofline(name, stats, ops, kernel):
    """Achieved int8 MFMA rate of one kernel class: algorithmic ops (2 per
    weight per token) over the class's event-timed duration."""
    ms, launches, _ = stats
    if launches == 0 or ms <= 0:
        return None
    achieved = ops / (ms / 1000.0) / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 1), "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
            "frac": round(achieved / INT8_PEAK_TOPS, 4), "traffic": None, "kernel_class": name,
            "launches": launches, "avg_us": round(ms / launches * 1000.0, 2),
            "algorithmic_ops_per_step": int(ops), "kernel": kernel}


def cpu_baseline_mixed(d, sched, model_dir, artifact, rows, ctx_lens, prefill_len, chunk, threads):
    """Config 5 on the reference (oracle/_ref, built from its sources), which
    cannot mix decode rows and a prompt chunk (cpu_engine_scheduler.inl:64-80):
    its packed-step equivalent is one 64-row advance_batch plus the prefill of
    one chunk. Measured pieces, summed:
    - the 64-row advance_batch of the reference engine, timed at 16-token
      contexts (prefilling 64 prompts of ~4k tokens on the CPU takes far
      longer than the bench allows);
    - the reference attention kernel (causal_attention_decode_gqa_pairs under
      CpuExecutor, requests x query-head pairs) over the config's own 64
      contexts, once per full-attention layer: the part the short contexts
      leave out;
    - the reference engine's advance() prefill of the 4096-token prompt with
      prefill_chunk_size = chunk, per `chunk` tokens.
    All on `threads` pinned cores."""
    from oracle import q35_oracle as orc  # the checker build, timed as the baseline only

    if not orc.ref_available():
        log("oracle/_ref not built: no config-5 CPU baseline")
        return None
    r = orc.ref()
    with open(os.path.join(model_dir, "config.json"), "w") as f:
        json.dump(CONFIG_4B, f)
    cpus, cpu_model, allowed, physical = host_cpus(threads)
    threads = len(cpus)
    before = os.sched_getaffinity(0)
    os.sched_setaffinity(0, cpus)
    isa = r.ref_backend_name(r.ref_backend_resolve(0)).decode()
    rng = np.random.default_rng(4243)
    short = 16
    dprompts = rng.integers(0, d.vocab, size=(rows, short)).astype(np.int32)
    prompt = rng.integers(0, d.vocab, size=prefill_len).astype(np.int32)
    dms, pms, calls = ctypes.c_double(), ctypes.c_double(), ctypes.c_size_t()
    err = ctypes.create_string_buffer(512)
    t = time.time()
    try:
        rc = r.ref_engine_mixed(os.fsencode(model_dir), os.fsencode(artifact), threads, dprompts.ctypes.data, short,
                                rows, prompt.ctypes.data, prefill_len, chunk, ctypes.byref(dms), ctypes.byref(pms),
                                ctypes.byref(calls), err, 512)
        if rc != 0:
            log(f"reference engine failed: {err.value.decode(errors='replace')}")
            return None
        # the attention over the config's contexts, every full layer
        heads, kvh, hd = d.n_heads, d.n_kv_heads, d.head_dim
        lens = ctx_lens.astype(np.int32)
        total = int(lens.sum())
        kv = rng.standard_normal((2, total, kvh * hd)).astype(np.float16).view(np.uint16)
        kptr = (ctypes.c_void_p * total)(*[kv[0, i].ctypes.data for i in range(total)])
        vptr = (ctypes.c_void_p * total)(*[kv[1, i].ctypes.data for i in range(total)])
        offs = np.concatenate([[0], np.cumsum(lens)[:-1]])
        krow = (ctypes.c_void_p * rows)(*[ctypes.addressof(kptr) + int(o) * 8 for o in offs])
        vrow = (ctypes.c_void_p * rows)(*[ctypes.addressof(vptr) + int(o) * 8 for o in offs])
        qv = rng.standard_normal((rows, heads * hd)).astype(np.float32)
        gates = rng.standard_normal((rows, heads * hd)).astype(np.float32)
        out = np.empty((rows, heads * hd), np.float32)
        stride = int(lens.max())
        scores = np.empty(rows * (heads // 2) * stride * heads, np.float32)
        ex = r.ref_executor_create(threads)
        full_layers = int(sum(1 for x in sched if not x))
        t0 = time.perf_counter()
        for _ in range(full_layers):
            r.ref_par_attention(ex, qv.ctypes.data, gates.ctypes.data, ctypes.addressof(krow), ctypes.addressof(vrow),
                                lens.ctypes.data, scores.ctypes.data, out.ctypes.data, rows, stride, heads, kvh, hd,
                                1.0 / np.sqrt(hd), 0)
        attn_ms = (time.perf_counter() - t0) * 1000
        r.ref_executor_destroy(ex)
    finally:
        os.sched_setaffinity(0, before)
    step_ms = dms.value + attn_ms + pms.value * chunk / prefill_len
    value = (rows + chunk) / step_ms * 1000.0
    log(f"reference CPU config 5: {rows}-row advance_batch {dms.value:.1f} ms (16-token contexts) + attention over "
        f"the config's contexts {attn_ms:.1f} ms ({full_layers} layers) + {prefill_len}-token prefill "
        f"{pms.value:.0f} ms in {calls.value} advance() calls -> {step_ms:.1f} ms per {rows} + {chunk} tokens, "
        f"{value:.1f} tok/s on {threads} threads ({cpu_model}, {isa}) ({time.time() - t:.1f}s wall)")
    return {"value": round(value, 2), "unit": "tokens/s", "cores": threads, "kind": "reference",
            "cpu_model": cpu_model, "isa": isa, "threads": threads, "pinned_cpus": cpus,
            "decode_step_ms": round(dms.value, 2), "attention_ms": round(attn_ms, 2),
            "prefill_ms": round(pms.value, 1), "prefill_advance_calls": int(calls.value),
            "sample": f"reference engine: one {rows}-row advance_batch (max_decode_batch_size {rows}) at 16-token "
                      f"contexts, plus the reference attention kernel over the config's {rows} contexts (sum "
                      f"{total}) for each of {full_layers} full layers, plus the advance() prefill of a "
                      f"{prefill_len}-token prompt with prefill_chunk_size {chunk}, counted per {chunk} tokens; "
                      f"value = ({rows} + {chunk}) tokens / that sum"}


def run_mixed4b(args, q, ctx):
    """Config 5: the 4B-shaped model (hidden 2560, 32 layers 3:1, MLP 9216,
    random-init Q4) with 64 decode requests at contexts ~U[128, 8192] and one
    4096-token prompt, packed into one step per prompt chunk
    (q35_runtime_step_segments: the 64 decode rows plus `--prefill-chunk`
    prompt positions per step). Measured beside it, the reference's
    alternating schedule (cpu_engine_scheduler.inl:64-80: a 64-row decode step,
    captured graph, then the prompt chunk on its own) and the prompt's chunked
    prefill alone. Every shape the timed region uses runs once untimed first
    (graph capture and instantiation stay out of the timings). Decode cost does
    not depend on KV values, so the 64 rows' pages are allocated to their
    context lengths without running their prompts."""
    d, sched = q.model_dims(2)
    path = os.path.join(tempfile.gettempdir(), f"q35_bench_4b_s{args.seed}")
    os.makedirs(path, exist_ok=True)
    art = os.path.join(path, "model.q35h128")
    if not os.path.exists(art):
        t = time.time()
        log("writing the random-init 4B artifact (about a minute)")
        q.write_random_artifact(art + ".part", d, sched, seed=args.seed, weight_std=0.02)
        os.replace(art + ".part", art)
        log(f"wrote {art} ({os.path.getsize(art) / 1e9:.2f} GB) in {time.time() - t:.1f}s")
    t = time.time()
    model = q.Model(ctx, d, sched, artifact=art)
    log(f"4B model resident in HBM in {time.time() - t:.1f}s")
    rows, prefill_len, page_tokens, chunk = 64, 4096, 16, args.prefill_chunk
    n_chunks = (prefill_len + chunk - 1) // chunk
    rng = np.random.default_rng(20261205)
    ctx_lens = rng.integers(128, 8193, size=rows)
    steps = max(1, min(args.steps, 40))
    # decode positions written per row: warm-up and timed decode steps, two
    # rounds of packed steps (untimed, timed), the profiled steps
    advance = args.warmup + steps + 2 * n_chunks + 3
    max_ctx = 8192 + advance + 8
    rt = q.Runtime(model, max_slots=rows + 4, max_batch=rows, max_context=max_ctx, page_tokens=page_tokens,
                   use_graphs=args.graphs == "on", max_step_rows=rows + chunk)
    slots = np.array([rt.slot_alloc(np.array([1], np.int32)) for _ in range(rows)], np.int32)
    table = np.zeros((rows, rt.max_pages), np.int32)
    for r in range(rows):
        # positions ctx - 1 .. ctx - 2 + advance are written
        need = (int(ctx_lens[r]) + advance - 2) // page_tokens + 1
        assert need <= rt.max_pages
        for p in range(need):
            table[r, p] = rt.page_alloc()
    tokens = rng.integers(0, d.vocab, size=rows).astype(np.int32)
    pos = ctx_lens.astype(np.int32) - 1
    ones = np.ones(rows, np.uint8)
    for _ in range(args.warmup):
        tokens = rt.step(slots, pos, tokens, table, count_input=ones)
        pos += 1
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        tokens = rt.step(slots, pos, tokens, table, count_input=ones)
        pos += 1
    decode_ms = (time.perf_counter() - t0) * 1000 / steps
    log(f"4B decode: {rows} rows, contexts {int(ctx_lens.min())}..{int(ctx_lens.max())} "
        f"(sum {int(ctx_lens.sum())}): {decode_ms:.3f} ms/step")

    prompt = rng.integers(0, d.vocab, size=prefill_len).astype(np.int32)

    def prompt_slot():
        pslot = rt.slot_alloc(prompt)
        ptable = np.zeros(rt.max_pages, np.int32)
        for p in range(prefill_len // page_tokens + 1):
            ptable[p] = rt.page_alloc()
        return pslot, ptable

    def release(pslot, ptable):
        rt.slot_free(pslot)
        for p in range(prefill_len // page_tokens + 1):
            rt.page_release(int(ptable[p]))

    def prefill_alone():
        """The prompt alone, in chunks (the alternating schedule's prefill steps)."""
        pslot, ptable = prompt_slot()
        ctx.synchronize()
        t0 = time.perf_counter()
        first = None
        for c0 in range(0, prefill_len, chunk):
            first = rt.prefill(pslot, c0, prompt[c0:c0 + chunk], ptable)
        ms = (time.perf_counter() - t0) * 1000
        release(pslot, ptable)
        return ms, first

    def packed(n=n_chunks):
        """The prompt packed with the 64 decode rows, one step per chunk."""
        nonlocal tokens
        pslot, ptable = prompt_slot()
        ctx.synchronize()
        t0 = time.perf_counter()
        first = None
        for c0 in range(0, n * chunk, chunk):
            last = c0 + chunk >= prefill_len
            segs = [dict(slot=int(slots[r]), pos0=int(pos[r]), tokens=tokens[r:r + 1], page_table=table[r],
                         count_input=1) for r in range(rows)]
            segs.append(dict(slot=pslot, pos0=c0, tokens=prompt[c0:c0 + chunk], page_table=ptable,
                             want_token=int(last)))
            out = rt.step_segments(segs)
            tokens = out[:rows].astype(np.int32)
            pos[:] += 1
            if last:
                first = int(out[rows])
        ms = (time.perf_counter() - t0) * 1000 / n
        release(pslot, ptable)
        return ms, first

    prefill_alone()  # untimed: every prefill chunk shape
    packed()         # untimed: every packed step shape
    prefill_ms, first_alone = prefill_alone()
    log(f"4B chunked prefill: {prefill_len} tokens in {n_chunks} chunks of {chunk}: {prefill_ms:.1f} ms "
        f"({prefill_len / prefill_ms * 1000:.0f} tok/s), first token {first_alone}")
    packed_ms, first_packed = packed()
    assert first_packed == first_alone, (first_packed, first_alone)
    alternating_ms = decode_ms + prefill_ms / n_chunks
    log(f"4B packed step: {rows} decode rows + {chunk} prompt positions: {packed_ms:.2f} ms/step; alternating "
        f"(decode step + prompt chunk): {alternating_ms:.2f} ms; same first token {first_packed}")
    # rooflines: the decode attention (HBM) in a 64-row decode step, the dense
    # GEMM (int8 MFMA) in a packed step; eager launches with HIP events
    rt.set_profiling(True)
    rt.profile_reset()
    for _ in range(2):
        tokens = rt.step(slots, pos, tokens, table, count_input=ones)
        pos += 1
    prof_dec = rt.profile()
    rt.profile_reset()
    packed(1)
    prof_pack = rt.profile()
    rt.set_profiling(False)
    attn_roof = roofline("attention", prof_dec["attention"], None,
                         "attention_kernel<4> (decode rows: one workgroup per (64-token chunk, KV head, row), fp16 "
                         "MFMA scores and P*V over paged K/V)")
    ops = 2.0 * (rows + chunk) * projection_weights(d, sched)
    gemm_roof = mfma_roofline("gemm", prof_pack["gemm"], ops,
                              "gemm_dense_kernel<NT, true> (every projection of a packed step of "
                              f"{rows} + {chunk} rows: int8 MFMA over Q4 DOT4 tiles, fp32 block chain)")
    for name, roof in (("decode attention", attn_roof), ("packed dense GEMM", gemm_roof)):
        if roof:
            log(f"4B {name}: {roof['achieved']} {roof['unit']} = {roof['frac']:.3f} of peak "
                f"({roof['launches']} launches, {roof['avg_us']} us avg)")
    rt.close()
    model.close()
    base = None
    if args.cpu_baseline == "on":
        threads = args.cpu_threads or min(16, host_cpus(1 << 20)[3] or 1)
        base = cpu_baseline_mixed(d, sched, path, art, rows, ctx_lens, prefill_len, chunk, threads)
    value = (rows + chunk) / packed_ms * 1000
    line = {
        "metric": "config 5 packed step: 4B-shaped, 64 decode rows (ctx ~U[128,8192]) + a chunk of a 4096-token "
                  "prompt per step",
        "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": steps, "warmup": args.warmup, "ms_per_step": round(packed_ms, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "q4xi8->i32 (projections), f32 (DeltaNet, attention)",
        "data": "synthetic: random-init 4B-shaped weights N(0,0.02) packed to Q4-G32-DOT4 H128, random tokens",
        "config": {"workload": "config 5 (4B-shaped decode rows + chunked prefill packed into one step)",
                   "decode_rows": rows, "decode_context_sum": int(ctx_lens.sum()), "prefill_tokens": prefill_len,
                   "prefill_chunk": chunk, "packed_ms_per_step": round(packed_ms, 3),
                   "alternating_ms_per_step": round(alternating_ms, 3), "decode_ms": round(decode_ms, 3),
                   "prefill_alone_ms": round(prefill_ms, 2)},
        "roofline": gemm_roof, "decode_attention_roofline": attn_roof, "cpu_baseline": base,
    }
    if base:
        line["speedup_vs_cpu_baseline"] = round(value / base["value"], 1)
    return line


def run_prefix0p8b(args, q, ctx):
    """Prefix cache (register_prefix / CpuRequestSpec::prefix) on the 0.8B
    model: 16 requests whose 512-token prompts share a 448-token prefix, each
    prefilled to its first token. Cold: every prompt prefilled in full; warm:
    the prefix is restored from its snapshot (state copy, shared KV pages) and
    only the 64 unique tokens are prefilled. The first tokens of both runs must
    be equal (a hit is bit-identical to a full prefill)."""
    d, sched, _, artifact = prepare_model_dir(q, args.seed, 0.02)
    model = q.Model(ctx, d, sched, artifact=artifact)
    rows, shared_len, total = 16, 448, 512
    rng = np.random.default_rng(20261206)
    shared = rng.integers(0, d.vocab, size=shared_len).astype(np.int32)
    prompts = [np.concatenate([shared, rng.integers(0, d.vocab, size=total - shared_len).astype(np.int32)])
               for _ in range(rows)]

    def run(prefix):
        eng_ids = [eng.submit(p, 1, prefix=prefix) for p in prompts]
        ctx.synchronize()
        t0 = time.perf_counter()
        eng.prefill_batch(eng_ids)
        ctx.synchronize()
        ms = (time.perf_counter() - t0) * 1000
        res = [eng.result(i) for i in eng_ids]
        for i in eng_ids:
            eng.release(i)
        return ms, [int(t[0]) for _, t in res], [r.prefix_restore_ms for r, _ in res]

    eng = q.Engine(model, max_resident_requests=rows + 1, max_context=total + 8, max_decode_batch_size=64,
                   page_tokens=16, use_graphs=False)
    run(0)  # warm-up: kernels loaded, pages touched
    cold_ms, cold_tok, _ = run(0)
    t0 = time.perf_counter()
    h = eng.register_prefix(shared, "bench")
    build_ms = (time.perf_counter() - t0) * 1000
    warm_ms, warm_tok, restore = run(h)
    eng.release_prefix(h)
    stats = eng.prefix_stats()
    eng.close()
    model.close()
    if warm_tok != cold_tok:
        raise RuntimeError(f"prefix hit tokens {warm_tok} differ from full prefill {cold_tok}")
    log(f"prefix: cold prefill {cold_ms:.1f} ms, prefix build {build_ms:.1f} ms, warm prefill {warm_ms:.1f} ms "
        f"(restore {np.mean(restore):.2f} ms per request); first tokens equal")
    return {
        "metric": "prompt tokens/s, 16 x 512-token prompts sharing a 448-token prefix (0.8B, prefix cache hit)",
        "value": round(rows * total / warm_ms * 1000, 1), "unit": "tokens/s", "n_gpus": 1, "steps": 1, "warmup": 1,
        "ms_per_step": round(warm_ms, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4xi8->i32 (projections), f32 (DeltaNet, attention)",
        "data": "synthetic: random-init 0.8B weights, random-token prompts",
        "config": {"workload": "prefix cache: shared 448-token prefix + 64 unique tokens per request",
                   "requests": rows, "cold_prefill_ms": round(cold_ms, 2), "prefix_build_ms": round(build_ms, 2),
                   "warm_prefill_ms": round(warm_ms, 2), "restore_ms_per_request": round(float(np.mean(restore)), 3),
                   "first_tokens_equal": True, "prefix_hits": stats["prefix_hits"]},
        "roofline": None, "cpu_baseline": None,
    }


def run_kernels(args, q, ctx):
    """Configs 1-3 at kernel level, each entry point called on its own
    (median of HIP-event brackets around single calls, so a figure is the
    call's kernels plus their launch gaps; pure kernel durations come from
    rocprofv3). Beside each, the reference's own kernel (oracle/_ref, one host
    thread, and on all physical cores under the reference's CpuExecutor, the
    way its engine partitions the work) on the same inputs. Algorithmic bytes
    as in the reference's
    q4_dot4 / delta_net / full_attention tests' shapes:
      config 1: W 3584 x 1024 DOT4 (2,064,384 B), 512 distinct copies rotated,
                X1 (B=1) and X4 (B=16) activations, fp32 outputs;
      config 2: DeltaNet B=16 x 16 heads x 128 x 128 fp32 state read + written;
      config 3: paged GQA attention B=16, contexts ~U[64, 4096], 8/2 heads,
                head_dim 256, fp16 K/V in shuffled 16-token pages."""
    sys.path.insert(0, ROOT)
    from oracle import q35_oracle as orc
    rng = np.random.default_rng(20261207)
    res = {}

    def gpu_us(call, reps):
        times = []
        for i in range(reps):
            ctx.synchronize()
            ctx.timer_begin()
            call(i)
            times.append(ctx.timer_end() * 1000.0)
        return float(np.median(times))

    def cpu_us(call, reps):
        t = time.perf_counter()
        for i in range(reps):
            call(i)
        return (time.perf_counter() - t) / reps * 1e6

    ref = orc.ref() if orc.ref_available() else None
    threads = args.cpu_threads or min(16, host_cpus(1 << 20)[3] or 1)
    cpus, cpu_model, _, _ = host_cpus(threads)
    exe = ref.ref_executor_create(len(cpus)) if ref is not None else None
    before = os.sched_getaffinity(0)

    def cpu_all_us(call, reps):
        """`call` on the pinned cores (the executor's workers inherit the
        process's affinity); one untimed call first."""
        os.sched_setaffinity(0, cpus)
        try:
            call(0)
            return cpu_us(call, reps)
        finally:
            os.sched_setaffinity(0, before)

    # ---- config 1
    rows, cols, copies = 3584, 1024, 512
    nb = cols // 32
    canon = orc.random_q4_blocks(rng, rows, cols)
    packed = orc.dot4_pack(canon, rows, nb)
    wbytes = packed.nbytes
    dw = ctx.array(shape=(copies * wbytes,), dtype=np.uint8)
    for c in range(copies):
        q.lib.q35_memcpy_h2d(ctx.handle, dw.address + c * wbytes, packed.ctypes.data, wbytes)
    ctx.synchronize()
    for B in (1, 16):
        x = rng.standard_normal((B, cols)).astype(np.float32)
        act = orc.q8_quantize_1(x[0]) if B == 1 else orc.h128_prepare_4(x)
        da = ctx.array(act)
        out = ctx.array(shape=(B, rows), dtype=np.float32)
        if B == 1:
            call = lambda i: q.lib.q35_q4_dot4_matvec(ctx.handle, dw.address + (i % copies) * wbytes, da.address,
                                                      out.address, rows, nb)
        else:
            call = lambda i: q.lib.q35_q4_dot4_matmul(ctx.handle, dw.address + (i % copies) * wbytes, da.address,
                                                      out.address, rows, B, nb, rows)
        us = gpu_us(call, copies)
        nbytes = wbytes + B * cols * 4 + B * rows * 4
        entry = {"gpu_us_per_call": round(us, 2), "algorithmic_bytes": nbytes,
                 "gpu_GBps": round(nbytes / us / 1e3, 1)}
        if ref is not None:
            ho = np.empty((B, rows), np.float32)
            if B == 1:
                c_us = cpu_us(lambda i: ref.ref_q4_dot4_matvec(packed.ctypes.data, act.ctypes.data, ho.ctypes.data,
                                                               rows, nb, 0), 200)
            else:
                c_us = cpu_us(lambda i: ref.ref_q4_dot4_matmul(packed.ctypes.data, act.ctypes.data, ho.ctypes.data,
                                                               rows, B, nb, rows, 0), 100)
            entry["cpu_us_per_call_1thread"] = round(c_us, 1)
            # all cores: 8-row DOT4 tiles under CpuExecutor
            entry["cpu_us_per_call_all_cores"] = round(cpu_all_us(
                lambda i: ref.ref_par_q4_dot4(exe, packed.ctypes.data, act.ctypes.data, ho.ctypes.data, rows, B, nb,
                                              0), 400), 1)
        res[f"config1_B{B}"] = entry
        log(f"config 1 B={B}: {entry}")
    dw.free()
    # ---- config 2 (one step; chained steps repeat it on the updated state)
    B, H, D = 16, 16, 128
    state = (rng.standard_normal((B, H, D, D)) * 0.02).astype(np.float32)
    ds = ctx.array(state)
    ptrs = ctx.array(np.array([ds.address + b * H * D * D * 4 for b in range(B)], np.uint64))

    def l2n(a):
        return (a / np.linalg.norm(a, axis=-1, keepdims=True)).astype(np.float32)

    qq = l2n(rng.standard_normal((B, H, D)))
    kk = l2n(rng.standard_normal((B, H, D)))
    vv = rng.standard_normal((B, H, D)).astype(np.float32)
    be = (1 / (1 + np.exp(-rng.standard_normal((B, H))))).astype(np.float32)
    al = np.exp(-np.log1p(np.exp(rng.standard_normal((B, H))))).astype(np.float32)
    bufs = [ctx.array(a) for a in (qq, kk, vv, al, be)]
    out = ctx.array(shape=(B, H, D), dtype=np.float32)
    us = gpu_us(lambda i: q.gated_delta_net_update_batch(ctx, ptrs, *bufs, out, B, H, D, D), 64)
    nbytes = 2 * B * H * D * D * 4 + 4 * B * H * D * 4 + 2 * B * H * 4
    entry = {"gpu_us_per_step": round(us, 2), "algorithmic_bytes": nbytes, "gpu_GBps": round(nbytes / us / 1e3, 1)}
    if ref is not None:
        hs, ho = state.copy(), np.empty((B, H, D), np.float32)

        def one(i):
            for b in range(B):
                ref.ref_gated_delta_net_update_rows(hs[b].ctypes.data, qq[b].ctypes.data, kk[b].ctypes.data,
                                                    vv[b].ctypes.data, al[b].ctypes.data, be[b].ctypes.data,
                                                    ho[b].ctypes.data, H, D, D, 0, H * D, 0)
        entry["cpu_us_per_step_1thread"] = round(cpu_us(one, 5), 1)
        sp = (ctypes.c_void_p * B)(*[hs[b].ctypes.data for b in range(B)])
        entry["cpu_us_per_step_all_cores"] = round(cpu_all_us(
            lambda i: ref.ref_par_delta(exe, ctypes.addressof(sp), qq.ctypes.data, kk.ctypes.data, vv.ctypes.data,
                                        al.ctypes.data, be.ctypes.data, ho.ctypes.data, B, H, D, D, 0), 20), 1)
    res["config2_B16"] = entry
    log(f"config 2: {entry}")
    # ---- config 3
    heads, kvh, hd, pt = 8, 2, 256, 16
    lens = rng.integers(64, 4097, size=16).astype(np.int32)
    pages = [(n + pt - 1) // pt for n in lens]
    perm = rng.permutation(sum(pages)).astype(np.int32)
    table = np.zeros((16, max(pages)), np.int32)
    o = 0
    for b in range(16):
        table[b, :pages[b]] = perm[o:o + pages[b]]
        o += pages[b]
    kp = rng.standard_normal((sum(pages), pt, kvh * hd)).astype(np.float16).view(np.uint16)
    vp = rng.standard_normal((sum(pages), pt, kvh * hd)).astype(np.float16).view(np.uint16)
    qv = rng.standard_normal((16, heads * hd)).astype(np.float32)
    gates = rng.standard_normal((16, heads * hd)).astype(np.float32)
    dq, dg, dk, dv, dt, dl = (ctx.array(a) for a in (qv, gates, kp, vp, table, lens))
    out = ctx.array(shape=(16, heads * hd), dtype=np.float32)
    us = gpu_us(lambda i: q.attention_decode_paged(ctx, dq, dg, dk, dv, dt, table.shape[1], dl, pt, out, 16, heads,
                                                   kvh, hd, 1.0 / 16.0), 64)
    nbytes = int(lens.sum()) * kvh * hd * 2 * 2 + 16 * heads * hd * 4 * 3
    entry = {"gpu_us_per_call": round(us, 2), "context_sum": int(lens.sum()), "algorithmic_bytes": nbytes,
             "gpu_GBps": round(nbytes / us / 1e3, 1)}
    if ref is not None:
        ho = np.empty((16, heads * hd), np.float32)
        scores = np.empty(int(lens.max()) * heads, np.float32)
        krows, vrows = [], []
        for b in range(16):
            kr = (ctypes.c_void_p * int(lens[b]))(*[kp[table[b, t // pt], t % pt].ctypes.data for t in range(lens[b])])
            vr = (ctypes.c_void_p * int(lens[b]))(*[vp[table[b, t // pt], t % pt].ctypes.data for t in range(lens[b])])
            krows.append(kr)
            vrows.append(vr)

        def one(i):
            for b in range(16):
                ref.ref_causal_attention_decode_gqa_pairs(qv[b].ctypes.data, gates[b].ctypes.data,
                                                          ctypes.addressof(krows[b]), ctypes.addressof(vrows[b]),
                                                          scores.ctypes.data, ho[b].ctypes.data, int(lens.max()),
                                                          heads * hd, kvh * hd, int(lens[b]), heads, kvh, hd,
                                                          1.0 / 16.0, 0, heads // 2, 0)
        entry["cpu_us_per_call_1thread"] = round(cpu_us(one, 3), 1)
        krow = (ctypes.c_void_p * 16)(*[ctypes.addressof(k) for k in krows])
        vrow = (ctypes.c_void_p * 16)(*[ctypes.addressof(v) for v in vrows])
        pscores = np.empty(16 * (heads // 2) * int(lens.max()) * heads, np.float32)
        entry["cpu_us_per_call_all_cores"] = round(cpu_all_us(
            lambda i: ref.ref_par_attention(exe, qv.ctypes.data, gates.ctypes.data, ctypes.addressof(krow),
                                            ctypes.addressof(vrow), lens.ctypes.data, pscores.ctypes.data,
                                            ho.ctypes.data, 16, int(lens.max()), heads, kvh, hd, 1.0 / 16.0, 0),
            10), 1)
    res["config3_B16"] = entry
    if exe is not None:
        ref.ref_executor_destroy(exe)
        res["cpu"] = {"threads_all_cores": len(cpus), "pinned_cpus": cpus, "cpu_model": cpu_model,
                      "isa": ref.ref_backend_name(ref.ref_backend_resolve(0)).decode()}
    log(f"config 3: {entry}")
    return {
        "metric": "kernel-level configs 1-3: per-call GPU latency and algorithmic HBM GB/s (1 GPU)",
        "value": res["config1_B16"]["gpu_GBps"], "unit": "GB/s (config 1, B=16)", "n_gpus": 1, "steps": 1,
        "warmup": 0, "ms_per_step": round(res["config1_B16"]["gpu_us_per_call"] / 1000, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4xi8->i32 (config 1), f32 (configs 2, 3)", "data": "synthetic, seeded",
        "config": {"workload": "kernel-level configs 1-3", **res}, "roofline": None, "cpu_baseline": None,
    }


def roofline(name, stats, traffic, kernel=None):
    """Achieved HBM rate of one kernel class: algorithmic bytes per launch over
    the average launch duration (HIP events around each launch on the
    runtime's stream)."""
    ms, launches, nbytes = stats
    if launches == 0 or ms <= 0:
        return None
    per_launch_bytes = nbytes / launches
    per_launch_s = ms / launches / 1000.0
    achieved = per_launch_bytes / per_launch_s / 1e9
    t = traffic.get(name) if traffic else None
    measured = t.get("bytes_per_launch") if isinstance(t, dict) else None
    out = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured,
           "kernel_class": name, "launches": launches, "avg_us": round(ms / launches * 1000.0, 2),
           "algorithmic_bytes_per_launch": round(per_launch_bytes)}
    if measured:
        # HBM bytes the rocprofv3 PMC passes measured per launch of this class
        # (FETCH_SIZE + WRITE_SIZE, scaled by a copy kernel of known size)
        # over the algorithmic bytes: above 1 is split partials and re-reads
        out["traffic_vs_algorithmic"] = round(measured / per_launch_bytes, 3)
        out["traffic_source"] = "profiles/traffic.json (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs of this build)"
    if kernel:
        out["kernel"] = kernel
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=119, help="timed decode forwards")
    ap.add_argument("--warmup", type=int, default=8, help="untimed decode forwards")
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--profile-steps", type=int, default=16, help="decode forwards in the profiled region")
    ap.add_argument("--timing-steps", type=int, default=16,
                    help="decode forwards after the timed region whose graph replays are bracketed by HIP events")
    ap.add_argument("--cpu-baseline", choices=("on", "off"), default="on")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="0 = one per physical core of the allowed CPUs, at most 16 (the box's CPU share)")
    ap.add_argument("--cpu-tokens", type=int, default=128, help="greedy tokens per request in the CPU sample")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--prefill-chunk", type=int, default=2048, help="mixed4b: prompt positions per packed step")
    ap.add_argument("--calibration-copy-mb", type=int, default=0,
                    help="issue one device-to-device copy of this many MiB (a known-size kernel for HBM counters)")
    ap.add_argument("--workload", choices=("decode0p8b", "mixed4b", "prefix0p8b", "kernels"), default="decode0p8b",
                    help="decode0p8b: the headline metric (config 4); mixed4b: config 5; "
                         "prefix0p8b: prefill with a prefix-cache hit")
    ap.add_argument("--encodings", choices=("q4", "g16q8"), default="q4",
                    help="decode0p8b artifact: Q4 throughout, or the G16 tied head with Q8_0 gate rows")
    ap.add_argument("--graphs", choices=("on", "off"), default="on",
                    help="replay captured step graphs (off: eager launches, e.g. under rocprofv3)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}, WORLD_SIZE {world})", file=sys.stderr)
        sys.exit(2)
    if args.steps <= 0 or args.warmup < 0 or args.batch <= 0 or args.profile_steps < 0 or args.timing_steps < 0:
        ap.error("steps must be positive and warmup/profile-steps/timing-steps non-negative")

    import __graft_entry__ as entry

    q = entry.load()
    ctx = q.Context(0)
    cu, arch = ctx.device_info()
    log(f"device {arch}, {cu} CUs")
    if args.workload != "decode0p8b":
        runs = {"mixed4b": run_mixed4b, "prefix0p8b": run_prefix0p8b, "kernels": run_kernels}
        line = runs[args.workload](args, q, ctx)
        ctx.close()
        print(json.dumps(line), flush=True)
        return
    d, sched, model_dir, artifact = prepare_model_dir(q, args.seed, 0.02, args.encodings)
    if args.calibration_copy_mb > 0:
        n = args.calibration_copy_mb << 20
        src, dst = ctx.array(shape=(n,), dtype=np.uint8), ctx.array(shape=(n,), dtype=np.uint8)
        ctx.check(q.lib.q35_memcpy_d2d(ctx.handle, dst.ptr, src.ptr, n), "calibration copy")
        ctx.synchronize()
        src.free()
        dst.free()
        log(f"calibration copy of {args.calibration_copy_mb} MiB done")

    t = time.time()
    model = q.Model(ctx, d, sched, artifact=artifact)
    log(f"model resident in HBM in {time.time() - t:.1f}s")
    total_new = 1 + args.warmup + args.steps + args.timing_steps + args.profile_steps
    engine = q.Engine(model, max_resident_requests=args.batch, max_context=args.prompt + total_new + 16,
                      max_decode_batch_size=args.batch, prefill_chunk_size=128, page_tokens=16, use_graphs=args.graphs == "on")
    rng = np.random.default_rng(20261201)
    prompts = rng.integers(0, d.vocab, size=(args.batch, args.prompt)).astype(np.int32)
    ids = [engine.submit(p, max_new_tokens=total_new) for p in prompts]
    t = time.time()
    engine.prefill_batch(ids)
    log(f"prefilled {args.batch} x {args.prompt} tokens in {time.time() - t:.2f}s")

    for _ in range(args.warmup):
        engine.advance_batch(ids)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        engine.advance_batch(ids)
    ctx.synchronize()
    elapsed = time.perf_counter() - t0
    tok_s = args.batch * args.steps / elapsed
    log(f"timed {args.steps} decode forwards: {elapsed * 1000 / args.steps:.3f} ms/step, {tok_s:.0f} tok/s")

    # the GPU time of the replayed step itself: each graph launch between two
    # HIP events (outside the timed region; the wall time of the same steps
    # beside it gives the host's share)
    step_gpu = None
    if args.timing_steps:
        engine.set_step_timing(True)
        t1 = time.perf_counter()
        for _ in range(args.timing_steps):
            engine.advance_batch(ids)
        ctx.synchronize()
        wall_ms = (time.perf_counter() - t1) * 1000.0
        gpu_ms, n = engine.step_timing()
        engine.set_step_timing(False)
        if n != args.timing_steps:
            raise SystemExit(f"step timing counted {n} of {args.timing_steps} steps")
        step_gpu = {"gpu_us_per_step": round(gpu_ms / n * 1000.0, 1), "wall_us_per_step": round(wall_ms / n * 1000.0, 1),
                    "host_us_per_step": round((wall_ms - gpu_ms) / n * 1000.0, 1), "steps": n,
                    "graphs": args.graphs == "on",
                    "source": "q35_runtime_set_step_timing: HIP events around each step's graph launch on its stream"}
        log(f"step timing: {step_gpu['gpu_us_per_step']} us of GPU time in {step_gpu['wall_us_per_step']} us per "
            f"step ({args.timing_steps} steps)")

    prof = {}
    if args.profile_steps:
        engine.profile_reset()
        engine.set_profiling(True)
        for _ in range(args.profile_steps):
            engine.advance_batch(ids)
        ctx.synchronize()
        engine.set_profiling(False)
        prof = engine.profile()
        step_ms = sum(v[0] for v in prof.values()) / args.profile_steps
        for name, (ms, n, by) in sorted(prof.items(), key=lambda kv: -kv[1][0]):
            if n:
                log(f"  {name:10s} {ms / args.profile_steps * 1000:9.1f} us/step  {n // args.profile_steps:4d} "
                    f"launches/step  {by / ms / 1e6 if ms else 0:8.1f} GB/s")
        log(f"  kernel time per step {step_ms * 1000:.1f} us (eager, events)")

    for rid in ids:
        res, toks = engine.result(rid)
        if toks.size != 1 + args.warmup + args.steps + args.timing_steps + args.profile_steps:
            raise SystemExit(f"request {rid} produced {toks.size} tokens")
    engine.close()
    model.close()
    ctx.close()

    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f)
    # the Q4 GEMV the metric names: the vocabulary head (248,320 x 1024 Q4,
    # 143 MB per launch, one launch per step); the per-layer projections are
    # reported beside it as one class
    # traffic.json keys carry the artifact encodings ("head", "head_g16q8")
    sfx = "" if args.encodings == "q4" else f"_{args.encodings}"
    head_name = ("head_kernel<4, 3, NT, true, *> (greedy head: streaming Q4 GEMV + penalty + argmax, NT token tiles)"
                 if not sfx else "head_kernel<4, 2, NT, true, *, true> (greedy G16 head: Q4G16Tile GEMV, per-half "
                 "MFMA dots + penalty + argmax)")
    head_roof = roofline("head" + sfx, prof["head"], traffic, head_name) if prof else None
    # the dominant kernel class: the per-layer Q4 projections (at B <= 16:
    # split-K launches, the out / o projection with its residual, and the
    # gate_up projection with the post-attention norm in its prologue)
    roof = roofline("gemm" + sfx, prof["gemm"], traffic,
                    "per-layer Q4 projections: gemm_rows_kernel<KS, RM> (in / qkv, down; split-K), "
                    "gemm_resid_kernel<BPS, W> (out / o, all K splits + residual in one workgroup), "
                    "gemm_norm_kernel<RM, NQ, BPS> (post-attention RMSNorm + H128 prologue, gate_up; split-K)") \
        if prof else None
    breakdown = ({k: {"us_per_step": round(v[0] / args.profile_steps * 1000.0, 1),
                      "launches_per_step": v[1] // args.profile_steps} for k, v in prof.items() if v[1]}
                 if prof else None)

    base = None
    if args.cpu_baseline == "on":
        threads = args.cpu_threads or min(16, host_cpus(1 << 20)[3] or 1)
        base = cpu_baseline(model_dir, artifact, args.batch, args.prompt, args.cpu_tokens, threads)

    line = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(elapsed * 1000 / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "q4xi8->i32 (projections), f32 (DeltaNet, attention)",
        "data": "synthetic: random-init weights N(0,0.02) packed to Q4-G32-DOT4 H128, random-token prompts" +
                ("" if args.encodings == "q4" else
                 "; tied head/embedding as Q4G16Tile (G16), linear_attn.in_proj_ba gate rows as Q8_0"),
        "config": {"workload": "random-init Qwen3.5-0.8B-shaped hybrid, batched greedy decode",
                   "batch": args.batch, "prompt_tokens": args.prompt, "encodings": args.encodings,
                   "decode_forwards_timed": args.steps, "graphs": args.graphs == "on"},
        "roofline": roof, "head_roofline": head_roof, "step_kernel_breakdown": breakdown, "step_gpu": step_gpu,
        "cpu_baseline": base,
    }
    if base:
        line["speedup_vs_cpu_baseline"] = round(tok_s / base["value"], 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
