"""Benchmark: MoE FFN tokens/s of the Qwen3-30B-A3B-shaped MoE stack on one MI355X.

Workload (the single 30B-A3B MoE layer, decode, Q8_0 experts, F16 router, repeated over the model's
48 MoE layers): one step runs the whole MoE block - router, top-8, permutation, gate/up GEMV +
SwiGLU, down GEMV, weighted combine, residual - of each of 48 layers for T tokens (T = 1 by default;
T = 8 is reported alongside). Every layer has its own HBM copy of the expert table (48 x 642 MB =
30.8 GB, so the 256 MB last-level cache cannot serve repeats), its own F16 router weights and its
own N(0, 1) hnorm rows. Weights are random-init and synthetic (seeded); one layer's expert bytes are
generated and uploaded into each layer's slots.

The timed region replays one captured HIP graph per step on torch's current stream, bracketed by
synchronize; value = T * steps / seconds (tokens/s through all 48 MoE layers).

Roofline: the dominant kernel is gate_up (two thirds of the bytes). Its average duration is measured
with HIP events recorded around each of its launches on the launch stream (the library's stage
timing, over `--steps` eager steps), and its algorithmic bytes per launch are the distinct experts'
gate+up bytes plus activations in and SwiGLU rows out.

prefill: the same layer with Q4_K experts as a 512-token prefill with a Zipf(1.1)-skewed router
(the grouped MFMA path), over 8 layer copies; reported beside the decode line with its own
roofline (algorithmic flops per second against the int8 MFMA peak, and expert bytes per second
against HBM).

stack235 (on by default, --no-stack235 skips it): the Qwen3-235B-A22B-shaped 94-layer Q4_K MoE stack at
batch 1, fully resident (~128 GB of HBM) and with the expert pool capped at 32 GiB (misses streamed from
pinned host memory; host acquire and device acquire).

model30b (on by default, --no-model30b skips it): the whole 30B-A3B-shaped model - attention, MoE
blocks and the 151936-token output head - decoding one sequence at a 4096-token KV context, T = 1, 8
and 32 tokens per step, each step a replay of the captured forward pass; and a 512-token prompt step.

cpu_baseline: a CPU restatement of ggml semantics (oracle/cpu_ggml.c: Q8_0 / Q8_K activations, int8
block dots with AVX-512 VNNI, OpenMP over (expert, row block); checked against the oracle by
tests/test_cpu_ggml.py) runs the same decode layer on the host cores for a bounded sample of layer
passes, each with new hnorm rows (so new experts), and the 512-token prefill layer for a few passes.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

H, F, E, K, N_LAYER = 2048, 768, 128, 8, 48
Q8_0 = 8
Q4_K = 12
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # dense MFMA int8, MI355X
FP16_PEAK_TFLOPS = 2500.0  # dense MFMA fp16, MI355X


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--tokens", type=int, default=1)
    ap.add_argument("--layers", type=int, default=N_LAYER)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--prefill-layers", type=int, default=8)
    ap.add_argument("--no-decode", action="store_true", help="skip the decode legs (profiling the prefill leg alone)")
    ap.add_argument("--no-stack235", action="store_true",
                    help="skip the Qwen3-235B-A22B-shaped 94-layer Q4_K stack (resident, ~128 GB of HBM, and with the "
                         "pool capped at --pool-gib GiB, misses streamed from the pinned host tier)")
    ap.add_argument("--stack235-layers", type=int, default=94)
    ap.add_argument("--pool-gib", type=int, default=32)
    ap.add_argument("--stream-tokens", type=int, default=8)
    ap.add_argument("--no-model30b", action="store_true",
                    help="skip the whole 30B-A3B-shaped model (attention + MoE + head) decoding at a long KV context")
    ap.add_argument("--model30b-layers", type=int, default=N_LAYER)
    ap.add_argument("--context", type=int, default=4096)
    ap.add_argument("--model30b-tokens", type=str, default="1,8,32", help="tokens per decode step, comma-separated")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="first run one device-to-device copy of this many MiB (the reference kernel that scales "
                         "rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes)")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Stack:
    """Resident pool of the 30B-A3B MoE layers plus per-layer inputs on the device."""

    def __init__(self, torch, L, n_layer, t_max, seed=0):
        from localstack_amd import synth
        self.torch = torch
        self.n_layer = n_layer
        rng = np.random.default_rng(seed)
        t0 = time.time()
        self.up = synth.experts(rng, Q8_0, E, F, H)
        self.gate = synth.experts(rng, Q8_0, E, F, H)
        self.down = synth.experts(rng, Q8_0, E, H, F)
        log(f"[bench] generated one layer of Q8_0 experts ({3 * self.up.nbytes / 1e9:.2f} GB) in {time.time() - t0:.1f}s")
        t0 = time.time()
        types = (Q8_0,) * 3
        self.store = L.ExpertStore(n_layer, H, F, E, K, t_max, [(types, self.up, self.gate, self.down)] * n_layer)
        log(f"[bench] resident pool: {self.store.total_bytes() / 1e9:.1f} GB in HBM, built in {time.time() - t0:.1f}s")
        dev = torch.device("cuda:0")
        d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        self.routers = [d(synth.router_f16(rng, E, H)) for _ in range(n_layer)]
        self.routers_host = None
        self.rng = rng
        self.dev = dev
        self.t_max = t_max

    def inputs(self, T, seed):
        from localstack_amd import synth
        torch = self.torch
        rng = np.random.default_rng(seed)
        d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(self.dev)
        self.T = T
        self.x = [d(synth.activations(rng, T, H)) for _ in range(self.n_layer)]
        self.resid = [d(synth.activations(rng, T, H)) for _ in range(self.n_layer)]
        self.out = [torch.zeros((T, H), dtype=torch.float32, device=self.dev) for _ in range(self.n_layer)]
        self.ids = [torch.zeros((T, K), dtype=torch.int32, device=self.dev) for _ in range(self.n_layer)]
        self.w = [torch.zeros((T, K), dtype=torch.float32, device=self.dev) for _ in range(self.n_layer)]

    def step(self):
        for l in range(self.n_layer):
            self.store.block(l, self.x[l], self.routers[l], 1, self.resid[l], self.out[l], self.ids[l], self.w[l])


def time_steps(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def step_percentiles(torch, fn, steps):
    """p10 / p50 / p90 of single-step times, from an event pair around each of `steps` further steps
    (a pass of its own, so the per-step events do not touch the timed run)."""
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    t = np.array([a.elapsed_time(b) for a, b in ev])
    return [float(np.percentile(t, q)) for q in (10, 50, 90)]


def measure(torch, st, T, steps, warmup, use_graph):
    st.inputs(T, seed=1000 + T)
    graph = None
    if use_graph:
        st.step()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            st.step()
        fn = graph.replay
    else:
        fn = st.step
    ms = time_steps(torch, fn, steps, warmup)
    pct = step_percentiles(torch, fn, steps)
    st.store.check()
    # stage timing (eager, events around every launch on the launch stream)
    st.store.set_timing(True)
    n_eager = max(2, min(steps, 10))
    for _ in range(n_eager):
        st.step()
    stage_ms, launches = st.store.timing()
    st.store.set_timing(False)
    ids = [i.cpu().numpy() for i in st.ids]
    distinct = np.array([len(np.unique(a)) for a in ids], np.float64)
    gu_bytes = distinct.mean() * 2 * 1671168 + T * (H + H // 32 * 8) + T * K * F * 4
    dn_bytes = distinct.mean() * 1671168 + T * K * (F * 4 + H * 4) + T * H * 8
    rt_bytes = E * H * 2 + T * H * 4
    avg = [stage_ms[i] / max(1, launches[i]) for i in range(4)]
    res = dict(T=T, ms_per_step=ms, tok_s=T * 1000.0 / ms, graph=use_graph, ms_per_step_p10_p50_p90=pct,
               stage_avg_us={"route": avg[0] * 1e3, "gate_up": avg[1] * 1e3, "down": avg[2] * 1e3,
                             "combine": avg[3] * 1e3},
               stage_launches=launches, distinct_experts_per_layer=float(distinct.mean()),
               bytes_per_layer=float(gu_bytes + dn_bytes + rt_bytes),
               gate_up_bytes=float(gu_bytes))
    res["layer_gbs"] = res["bytes_per_layer"] * st.n_layer / (ms * 1e-3) / 1e9
    res["gate_up_gbs"] = gu_bytes / (avg[1] * 1e-3) / 1e9
    return res, graph


def prefill_leg(torch, L, n_layer, T, steps, warmup):
    """The 30B-A3B MoE layer with Q4_K experts as a 512-token prefill with a Zipf(1.1)-skewed router:
    n_layer layer copies (340 MB of experts each, so replays rotate through more than the 256 MB
    last-level cache), one captured HIP graph of the n_layer MoE blocks per step."""
    from localstack_amd import synth
    rng = np.random.default_rng(11)
    t0 = time.time()
    up, gate, down = (synth.experts(rng, Q4_K, E, F, H), synth.experts(rng, Q4_K, E, F, H),
                      synth.experts(rng, Q4_K, E, H, F))
    store = L.ExpertStore(n_layer, H, F, E, K, T, [((Q4_K,) * 3, up, gate, down)] * n_layer)
    log(f"[bench] prefill pool: {store.total_bytes() / 1e9:.2f} GB of Q4_K experts, built in {time.time() - t0:.1f}s")
    dev = torch.device("cuda:0")
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    routers = [d(synth.zipf_router_f16(rng, E, H)) for _ in range(n_layer)]
    xs = [d(synth.activations(rng, T, H, bias_unit=True)) for _ in range(n_layer)]
    resid = [d(synth.activations(rng, T, H)) for _ in range(n_layer)]
    out = [torch.zeros((T, H), dtype=torch.float32, device=dev) for _ in range(n_layer)]
    ids = [torch.zeros((T, K), dtype=torch.int32, device=dev) for _ in range(n_layer)]
    w = [torch.zeros((T, K), dtype=torch.float32, device=dev) for _ in range(n_layer)]

    def step():
        for l in range(n_layer):
            store.block(l, xs[l], routers[l], 1, resid[l], out[l], ids[l], w[l])

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    ms = time_steps(torch, graph.replay, steps, warmup)
    store.check()
    store.set_timing(True)
    for _ in range(max(2, min(steps, 10))):
        step()
    stage_ms, launches = store.timing()
    store.set_timing(False)
    # stage 0 = route + top-k + permute (3 launches per block), 1 = gate_up, 2 = act quant + down, 3 = combine
    per_block = [stage_ms[i] / max(1, launches[i] // (1 if i in (1, 3) else (3 if i == 0 else 2))) for i in range(4)]
    counts = [np.bincount(i.cpu().numpy().ravel(), minlength=E) for i in ids]
    active = float(np.mean([np.count_nonzero(c) for c in counts]))
    flops = 2.0 * T * K * 3 * H * F
    flops_gu = 2.0 * T * K * 2 * H * F
    wbytes = active * 3 * 884736
    layer_s = ms * 1e-3 / n_layer
    gu_s = per_block[1] * 1e-3
    del graph
    # layer_tok_s: prompt tokens per second through ONE MoE layer (T tokens x n_layer layer copies per step); a
    # 48-layer model's prompt rate through its MoE blocks is layer_tok_s / 48
    return dict(T=T, n_layer=n_layer, ms_per_step=ms, layer_tok_s=T * n_layer / (ms * 1e-3), layer_us=layer_s * 1e6,
                stage_us_per_block={"route_topk_permute": per_block[0] * 1e3, "gate_up": per_block[1] * 1e3,
                                    "quant_down": per_block[2] * 1e3, "combine": per_block[3] * 1e3},
                active_experts=active, max_tokens_per_expert=int(max(c.max() for c in counts)),
                layer_tflops=flops / layer_s / 1e12, layer_hbm_gbs=wbytes / layer_s / 1e9,
                gate_up_tflops=flops_gu / gu_s / 1e12)


def stack235_leg(torch, L, n_layer, pool_gib, steps, warmup, stream_tokens):
    """The Qwen3-235B-A22B-shaped MoE stack (94 layers, h 4096, f 1536, 128 experts top-8, Q4_K,
    Zipf(1.1)-biased F16 router), batch-1 decode, two runs:
      resident   every expert of every layer in HBM (~128 GB): one captured HIP graph of the 94 MoE
                 blocks per token (router, top-8, gate/up + SwiGLU, down, combine, residual);
      streaming  the pool capped at pool_gib GiB (ExpertStore::init's slot split); per layer, in the
                 order of Engine::run_segment (src/engine.cpp:343-399): router on the device, ids to
                 the host, acquire (hits pin, misses evict the LRU head and are copied from the pinned
                 host tier on the pool's side streams), experts on the slots, release_all;
                 then the same with the acquire on the device (no host round trip), eager and as a
                 captured graph per token.
    One layer's expert bytes are generated and passed for every layer (the host tier then holds one
    copy); every layer has its own HBM slots, router weights and hnorm rows."""
    from localstack_amd import synth
    H5, F5 = 4096, 1536
    rng = np.random.default_rng(235)
    t0 = time.time()
    up, gate, down = (synth.experts(rng, Q4_K, E, F5, H5), synth.experts(rng, Q4_K, E, F5, H5),
                      synth.experts(rng, Q4_K, E, H5, F5))
    log(f"[bench] 235B stack: generated one layer of Q4_K experts ({3 * up.nbytes / 1e9:.2f} GB) in {time.time() - t0:.1f}s")
    dev = torch.device("cuda:0")
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    routers = [d(synth.zipf_router_f16(rng, E, H5)) for _ in range(n_layer)]
    mat = 3538944  # bytes of one Q4_K expert matrix at this shape
    layers = [((Q4_K,) * 3, up, gate, down)] * n_layer
    res = {"n_layer": n_layer, "n_embd": H5, "n_ff_exp": F5}
    # (i) resident
    t0 = time.time()
    store = L.ExpertStore(n_layer, H5, F5, E, K, 1, layers)
    log(f"[bench] 235B stack: resident pool {store.total_bytes() / 1e9:.1f} GB in HBM, built in {time.time() - t0:.1f}s")
    xs = [d(synth.activations(rng, 1, H5, bias_unit=True)) for _ in range(n_layer)]
    resid = [d(synth.activations(rng, 1, H5)) for _ in range(n_layer)]
    out = [torch.zeros((1, H5), dtype=torch.float32, device=dev) for _ in range(n_layer)]
    ids = [torch.zeros((1, K), dtype=torch.int32, device=dev) for _ in range(n_layer)]
    w = [torch.zeros((1, K), dtype=torch.float32, device=dev) for _ in range(n_layer)]

    def step():
        for l in range(n_layer):
            store.block(l, xs[l], routers[l], 1, resid[l], out[l], ids[l], w[l])

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    ms = time_steps(torch, graph.replay, steps, warmup)
    store.check()
    per_tok = n_layer * (K * 3 * mat + E * H5 * 2 + H5 * 8)
    res["resident"] = {"tok_s": 1000.0 / ms, "ms_per_token": ms, "bytes_per_token": per_tok,
                       "gbs": per_tok / (ms * 1e-3) / 1e9, "frac_hbm": per_tok / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                       "roofline": {"bound": "hbm", "achieved": per_tok / (ms * 1e-3) / 1e9, "peak": HBM_PEAK_GBS,
                                    "unit": "GB/s", "frac": per_tok / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                    "what": "94 layers x (8 routed Q4_K experts + F16 router + hnorm in/out) per token"},
                       "hbm_gb": store.total_bytes() / 1e9}
    del graph
    store.close()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    # (ii) streaming, pool capped at pool_gib GiB
    t0 = time.time()
    store = L.ExpertStore(n_layer, H5, F5, E, K, 1, layers, pool_bytes=pool_gib << 30, min_slots=2 * K + 2,
                          streaming=True)
    log(f"[bench] 235B stack: streaming pool {store.total_bytes() / 2**30:.1f} GiB, {store.total_slots()} slots, "
        f"built in {time.time() - t0:.1f}s")
    # every token routes new hnorm rows (2 warm-up tokens + the timed ones)
    n_tok = 2 + stream_tokens
    xs_tok = [[d(synth.activations(rng, 1, H5, bias_unit=True)) for _ in range(n_layer)] for _ in range(n_tok)]
    ids_h = torch.zeros((n_layer, K), dtype=torch.int32).pin_memory()
    slots_h = torch.zeros((n_layer, K), dtype=torch.int32).pin_memory()
    slots_d = torch.zeros((n_layer, K), dtype=torch.int32, device=dev)

    def token(xt):
        for l in range(n_layer):
            store.route(l, xt[l], routers[l], 1, ids[l], w[l])
            ids_h[l].copy_(ids[l][0])  # synchronous: the host needs the routing (as the reference does)
            slots_h[l] = torch.from_numpy(store.acquire(l, ids_h[l].numpy()))
            slots_d[l].copy_(slots_h[l], non_blocking=True)
            store.ffn(l, xt[l], slots_d[l:l + 1], w[l], resid[l], out[l])
            store.release_all()

    for i in range(2):
        token(xs_tok[i])
    torch.cuda.synchronize()
    s0 = store.stats()
    t0 = time.time()
    for i in range(stream_tokens):
        token(xs_tok[2 + i])
    torch.cuda.synchronize()
    el = time.time() - t0
    s1 = store.stats()
    hits, misses = s1["hits"] - s0["hits"], s1["misses"] - s0["misses"]
    rd = s1["bytes_read"] - s0["bytes_read"]
    res["streaming"] = {"pool_gib": pool_gib, "slots": store.total_slots(), "tokens": stream_tokens,
                        "tok_s": stream_tokens / el, "ms_per_token": el * 1e3 / stream_tokens,
                        "hit_rate": hits / max(1, hits + misses), "misses_per_token": misses / stream_tokens,
                        "host_to_hbm_gbs": rd / el / 1e9, "bytes_read_per_token": rd / stream_tokens}
    store.close()
    torch.cuda.synchronize()
    # (iii) streaming with the acquire on the device: the same pool size and token sequence, route ->
    # lstk_pool_acquire_device (resolve + copy kernels) -> experts, no host round trip; timed eager
    # and as one captured graph per token (the token's hnorm rows copied into the graph's inputs)
    store = L.ExpertStore(n_layer, H5, F5, E, K, 1, layers, pool_bytes=pool_gib << 30, min_slots=2 * K + 2,
                          streaming=True, device_lru=True)
    xs_g = [torch.zeros((1, H5), dtype=torch.float32, device=dev) for _ in range(n_layer)]

    def token_dev(xt):
        for l in range(n_layer):
            store.route(l, xt[l], routers[l], 1, ids[l], w[l])
            store.acquire_device(l, ids[l], slots_d[l:l + 1])
            store.ffn(l, xt[l], slots_d[l:l + 1], w[l], resid[l], out[l])

    def timed_tokens(run):
        for i in range(2):
            run(xs_tok[i])
        torch.cuda.synchronize()
        s0 = store.stats()
        t0 = time.time()
        for i in range(stream_tokens):
            run(xs_tok[2 + i])
        torch.cuda.synchronize()
        el = time.time() - t0
        s1 = store.stats()
        h_, m_ = s1["hits"] - s0["hits"], s1["misses"] - s0["misses"]
        rd_ = s1["bytes_read"] - s0["bytes_read"]
        return {"tok_s": stream_tokens / el, "ms_per_token": el * 1e3 / stream_tokens,
                "hit_rate": h_ / max(1, h_ + m_), "misses_per_token": m_ / stream_tokens,
                "host_to_hbm_gbs": rd_ / el / 1e9}

    res["streaming_device"] = timed_tokens(token_dev)
    store.check()
    store.close()
    # a fresh pool for the graph run, so it sees the same misses as the eager run
    store = L.ExpertStore(n_layer, H5, F5, E, K, 1, layers, pool_bytes=pool_gib << 30, min_slots=2 * K + 2,
                          streaming=True, device_lru=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        token_dev(xs_g)

    def token_graph(xt):
        for l in range(n_layer):
            xs_g[l].copy_(xt[l])
        graph.replay()

    res["streaming_device_graph"] = timed_tokens(token_graph)
    store.check()
    del graph
    store.close()
    return res


def model30b_leg(torch, L, n_layer, ctx, steps, warmup, t_list=(1, 8, 32)):
    """The whole Qwen3-30B-A3B-shaped model: 48 layers, h 2048, 32 query / 4 KV heads of 128, vocab
    151936 (head tied to the F16 embedding), 128 experts top-8 with f 768 as Q4_K (centred), F16
    attention and router, all resident in HBM. Decode of one sequence at a ctx-token KV context
    (synthetic: lstk_model_fill_context writes seeded K/V for ctx positions) with T in t_list tokens per
    step. One step = lstk_model_prepare (host KV bookkeeping and input upload) + the replay of a captured
    lstk_model_forward (every layer's attention and MoE block, the final norm and the output head).
    One layer's tensors are generated and uploaded into every layer's own HBM copies.
    Algorithmic HBM bytes per T=1 token: 48 x (attention weights + the K/V of ctx cells + router + 8
    experts) + the 151936 x 2048 head."""
    from localstack_amd import synth
    hp = dict(n_layer=n_layer, n_embd=H, n_head=32, n_head_kv=4, head_dim=128, n_vocab=151936, n_expert=E,
              n_expert_used=K, n_ff_exp=F, n_ctx_train=40960, rms_eps=1e-6, rope_freq_base=1e6)
    rng = np.random.default_rng(30)
    t0 = time.time()
    L0 = synth.qwen3_weights(rng, dict(hp, n_layer=1, n_vocab=8), wtype=Q4_K)["layers"][0]
    tok = (rng.standard_normal((hp["n_vocab"], H), dtype=np.float32) * np.float32(0.02)).astype(np.float16)
    w = {"tok_embd": tok, "output_norm": np.ones(H, np.float32), "output": None, "layers": [L0] * n_layer}
    t_max = max(t_list)
    n_prefill = 512
    nb = max(t_max, n_prefill)
    store = L.ExpertStore(n_layer, H, F, E, K, nb, [(L0["types"], L0["up"], L0["gate"], L0["down"])] * n_layer)
    kv = (ctx + t_max * (steps + warmup + 3) + 255) // 256 * 256
    dev = torch.device("cuda:0")
    model = L.Qwen3Model(hp, w, store, kv, nb, device=dev)
    del tok
    log(f"[bench] 30B model: {n_layer} layers built in {time.time() - t0:.1f}s, experts {store.total_bytes() / 1e9:.1f} GB, "
        f"KV cache {kv} cells")
    hq, hk = 32 * 128, 4 * 128
    attn_w = 2 * hq * H * 2 + 2 * hk * H * 2  # q and o (hq x H each), k and v (hk x H each), fp16 bytes
    kv_b = ctx * hk * 2 * 2
    expert_mat_b = F * (H // 256) * 144  # one Q4_K expert matrix (884,736 B)
    moe_b = E * H * 2 + K * 3 * expert_mat_b
    head_b = hp["n_vocab"] * H * 2
    per_tok = n_layer * (attn_w + kv_b + moe_b) + head_b
    res = {"n_layer": n_layer, "context": ctx, "bytes_per_token_T1": per_tok,
           "bytes_split_T1": {"attention_weights": n_layer * attn_w, "kv": n_layer * kv_b, "moe": n_layer * moe_b,
                              "head": head_b}}
    stream = torch.cuda.Stream()
    logits = torch.zeros(hp["n_vocab"], dtype=torch.float32, device=dev)
    for T in t_list:
        seq = T
        model.fill_context(seq, ctx, seed=T)
        # the attended cells of the last step: a forward over at least the prepared count is exact (cells
        # past a sequence's end are masked), so one capture serves the whole run
        n_cells = (ctx + T * (steps + warmup + 3) + 255) // 256 * 256
        toks = rng.integers(0, hp["n_vocab"], (steps + warmup + 4, T)).astype(np.int32)
        # per-stage device time from two eager steps (after one untimed step: the first multi-token step
        # loads the library GEMM's kernels)
        model.decode(seq, toks[-1], logits=logits)
        model.truncate_seq(seq, ctx)
        model.set_timing(True)
        store.set_timing(True)
        tr = torch.full((n_layer, T, K), -1, dtype=torch.int32, device=dev)
        for i in range(2):
            model.decode(seq, toks[i], logits=logits, trace=tr)
        torch.cuda.synchronize()
        distinct = distinct_experts(tr.cpu().numpy())
        mms, mn = model.timing()
        pms, pn = store.timing()
        model.set_timing(False)
        store.set_timing(False)
        with torch.cuda.stream(stream):
            model.prepare(seq, toks[2], stream=stream)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                model.forward(seq, T, n_cells, logits=logits, stream=stream)
            graph.replay()
            for i in range(warmup):
                model.prepare(seq, toks[3 + i], stream=stream)
                graph.replay()
            stream.synchronize()
            s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s_ev.record(stream)
            for i in range(steps):
                model.prepare(seq, toks[3 + warmup + i], stream=stream)
                graph.replay()
            e_ev.record(stream)
            stream.synchronize()
        ms = s_ev.elapsed_time(e_ev) / steps
        assert torch.isfinite(logits).all()
        stage = {"norms": mms[0] / 2, "qkv_rope": mms[1] / 2, "attention": mms[2] / 2, "o_proj": mms[3] / 2,
                 "head": mms[4] / 2, "moe_router": pms[0] / 2, "moe_gate_up": pms[1] / 2, "moe_down": pms[2] / 2,
                 "moe_combine": pms[3] / 2}
        moe_ms = sum(pms) / 2
        r = {"tok_s": T * 1000.0 / ms, "ms_per_step": ms, "steps": steps,
             "eager_stage_ms_per_step": stage, "moe_ms_per_step": moe_ms,
             "launches_per_step": (sum(mn) + sum(pn)) // 2, "seq_len_end": model.seq_len(seq)}
        # algorithmic HBM bytes of the step: every layer's attention weights, the K/V of the attended cells (read
        # once for all T tokens), the router and the distinct experts the step routed to; the head on one row
        ctx_now = ctx + T * (3 + warmup + steps // 2)
        step_b = n_layer * (attn_w + ctx_now * hk * 2 * 2 + E * H * 2 + distinct * 3 * expert_mat_b) + head_b
        r["bytes_per_step"] = step_b
        r["distinct_experts_per_layer"] = distinct
        r["gbs"] = step_b / (ms * 1e-3) / 1e9
        r["frac_hbm"] = r["gbs"] / HBM_PEAK_GBS
        r["roofline"] = {"bound": "hbm", "achieved": r["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": r["frac_hbm"],
                         "what": f"48 x (attention weights + K/V of ~{ctx_now} cells + router + "
                                 f"{distinct:.1f} distinct Q4_K experts) + head, per step of {T} tokens"}
        r["moe_gbs_eager"] = n_layer * (E * H * 2 + distinct * 3 * expert_mat_b) / (moe_ms * 1e-3) / 1e9
        res[f"T{T}"] = r
        log(f"[bench] 30B model T={T}: {json.dumps(r)}")
        del graph
        model.remove_seq(seq)
    # prompt processing: one 512-token step into an empty cache (eager: the step's host work included)
    prompt = rng.integers(0, hp["n_vocab"], n_prefill).astype(np.int32)
    times = []
    tr = torch.full((n_layer, n_prefill, K), -1, dtype=torch.int32, device=dev)
    for rep in range(3):
        torch.cuda.synchronize()
        t0 = time.time()
        model.decode(1000 + rep, prompt, logits=logits, trace=tr if rep == 0 else None)
        torch.cuda.synchronize()
        times.append(time.time() - t0)
        model.remove_seq(1000 + rep)
    ms = 1e3 * min(times[1:])
    active = distinct_experts(tr.cpu().numpy())
    # algorithmic work of the step: the MoE products on the int8 matrix cores; Q/K/V, o-proj, the causal
    # attention and the router in fp16 / f32; the head on the last row. Its roofline time is each part at
    # its own dense peak, and the effective peak is the step's flops over that time.
    T = n_prefill
    f_moe = n_layer * 2.0 * T * K * 3 * H * F
    f_dense = n_layer * (2.0 * T * (hq + 2 * hk) * H + 2.0 * T * hq * H + 4.0 * 32 * 128 * T * (T + 1) / 2 +
                         2.0 * T * H * E) + 2.0 * H * hp["n_vocab"]
    t_min = f_moe / (INT8_PEAK_TOPS * 1e12) + f_dense / (FP16_PEAK_TFLOPS * 1e12)
    tflops = (f_moe + f_dense) / (ms * 1e-3) / 1e12
    peak = (f_moe + f_dense) / t_min / 1e12
    pb = n_layer * (attn_w + T * hk * 2 * 2 + E * H * 2 + active * 3 * expert_mat_b) + head_b
    res["prefill512"] = {"tok_s": n_prefill * 1000.0 / ms, "ms": ms, "active_experts_per_layer": active,
                         "tflop_per_step": (f_moe + f_dense) / 1e12, "moe_share_of_flops": f_moe / (f_moe + f_dense),
                         "hbm_gbs": pb / (ms * 1e-3) / 1e9, "frac_hbm": pb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                         "roofline": {"bound": "mfma", "achieved": tflops, "peak": peak, "unit": "TFLOP/s",
                                      "frac": tflops / peak,
                                      "what": "the step's algorithmic flops; peak = those flops over their time at the "
                                              "dense MFMA peaks (MoE int8 5.0 POP/s, the rest fp16 2.5 PFLOP/s)"}}
    log(f"[bench] 30B model prefill {n_prefill}: {json.dumps(res['prefill512'])}")
    model.close()
    store.close()
    return res


def distinct_experts(trace):
    """Mean over layers of the distinct expert ids in a step's router trace [n_layer][T][k] (-1 = no row)."""
    return float(np.mean([len(np.unique(t[t >= 0])) for t in trace]))


def cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(T, seconds):
    """The CPU restatement of ggml semantics (oracle/cpu_ggml.c: Q8_0 / Q8_K activation quantization,
    int8 block dots with AVX-512 VNNI where the host has it, OpenMP over (expert, 16-row block)) on this
    host's cores: the decode layer (Q8_0, T tokens) for `seconds`, each pass with new hnorm rows so new
    experts stream from DRAM; then the 512-token Q4_K Zipf prefill layer for a few passes."""
    from oracle import cpu_ggml
    from localstack_amd import synth
    rng = np.random.default_rng(7)
    cores = len(os.sched_getaffinity(0))
    gate_inp = synth.router_f16(rng, E, H)
    xs = [synth.activations(rng, T, H) for _ in range(64)]
    resid = synth.activations(rng, T, H)
    up, gate, down = (synth.experts(rng, Q8_0, E, F, H), synth.experts(rng, Q8_0, E, F, H),
                      synth.experts(rng, Q8_0, E, H, F))
    cpu_ggml.moe_block(xs[0], gate_inp, up, gate, down, Q8_0, resid, E, F, K, n_threads=cores)
    n = 0
    t0 = time.time()
    while True:
        cpu_ggml.moe_block(xs[n % len(xs)], gate_inp, up, gate, down, Q8_0, resid, E, F, K, n_threads=cores)
        n += 1
        el = time.time() - t0
        if el >= seconds or n >= 100000:
            break
    per_layer = el / n
    # the same layer at T = 8 (config 2's second batch size), for a quarter of the time
    x8 = [synth.activations(rng, 8, H) for _ in range(16)]
    r8 = synth.activations(rng, 8, H)
    cpu_ggml.moe_block(x8[0], gate_inp, up, gate, down, Q8_0, r8, E, F, K, n_threads=cores)
    n8 = 0
    t0 = time.time()
    while True:
        cpu_ggml.moe_block(x8[n8 % len(x8)], gate_inp, up, gate, down, Q8_0, r8, E, F, K, n_threads=cores)
        n8 += 1
        el8 = time.time() - t0
        if el8 >= seconds / 4 or n8 >= 100000:
            break
    per_layer8 = el8 / n8
    del up, gate, down
    # prefill: 512 tokens, Q4_K experts, Zipf(1.1)-biased router (the GPU prefill leg's workload)
    up4, gate4, down4 = (synth.experts(rng, Q4_K, E, F, H), synth.experts(rng, Q4_K, E, F, H),
                         synth.experts(rng, Q4_K, E, H, F))
    zr = synth.zipf_router_f16(rng, E, H)
    xp = [synth.activations(rng, 512, H, bias_unit=True) for _ in range(2)]
    rp = synth.activations(rng, 512, H)
    m = 0
    t0 = time.time()
    while True:
        cpu_ggml.moe_block(xp[m % 2], zr, up4, gate4, down4, Q4_K, rp, E, F, K, n_threads=cores)
        m += 1
        pel = time.time() - t0
        if pel >= seconds / 2 or m >= 50:
            break
    pre_layer = pel / m
    return dict(value=T / (per_layer * N_LAYER), unit="tok/s", cores=cores, kind="port",
                label="CPU restatement of ggml semantics", cpu_model=cpu_model(), isa=cpu_ggml.isa(),
                sample=f"{n} passes of one Qwen3-30B-A3B MoE layer (router + Q8_0 experts, T={T}, new hnorm rows "
                       f"each pass) by oracle/cpu_ggml.c on {cores} threads, scaled to 48 layers; "
                       f"{per_layer * 1e3:.3f} ms per layer",
                t8={"value": 8 / (per_layer8 * N_LAYER), "unit": "tok/s", "ms_per_layer": per_layer8 * 1e3,
                    "passes": n8, "what": "the same layer at T=8 (new hnorm rows each pass), scaled to 48 layers"},
                prefill={"layer_tok_s": 512 / pre_layer, "ms_per_layer": pre_layer * 1e3, "passes": m,
                         "what": "512-token Q4_K Zipf(1.1) prefill through one MoE layer"})


def measured_traffic(key):
    """HBM bytes per launch of a kernel from the committed rocprofv3 PMC summary (FETCH_SIZE and
    WRITE_SIZE passes scaled by a plain copy of known size; the commands are in the file), or None."""
    path = os.path.join(ROOT, "profiles", "moe_decode_30b_q8_0_traffic.txt")
    try:
        with open(path) as fh:
            for line in fh:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == key:
                    return float(parts[2])
    except OSError:
        pass
    return None


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {a.gpus}); the multi-GPU expert-parallel path is not built.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import localstack_amd as L
    L.lib()
    if a.calibrate_copy_mib:
        n = a.calibrate_copy_mib << 18
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration copy: {a.calibrate_copy_mib} MiB read, {a.calibrate_copy_mib} MiB written")
        del src, dst
    if a.no_decode:
        out = {}
        if not a.no_prefill:
            out["prefill"] = prefill_leg(torch, L, a.prefill_layers, 512, max(5, a.steps // 5), 2)
        if not a.no_stack235:
            out["stack235"] = stack235_leg(torch, L, a.stack235_layers, a.pool_gib, max(5, a.steps // 2), 2,
                                           a.stream_tokens)
        if not a.no_model30b:
            out["model30b"] = model30b_leg(torch, L, a.model30b_layers, a.context, max(5, a.steps // 5), 2,
                                            tuple(int(t) for t in a.model30b_tokens.split(",")))
        print(json.dumps(out), flush=True)
        return
    st = Stack(torch, L, a.layers, t_max=max(8, a.tokens))
    main_res, g = measure(torch, st, a.tokens, a.steps, a.warmup, not a.no_graph)
    del g
    log(f"[bench] T={a.tokens}: {json.dumps(main_res)}")
    extra = None
    if a.tokens == 1:
        extra, g = measure(torch, st, 8, a.steps, a.warmup, not a.no_graph)
        del g
        log(f"[bench] T=8: {json.dumps(extra)}")
    pre = None
    if not a.no_prefill:
        pre = prefill_leg(torch, L, a.prefill_layers, 512, max(5, a.steps // 5), 2)
        log(f"[bench] prefill: {json.dumps(pre)}")
        pre["roofline"] = {"bound": "hbm", "note": "512-token Q4_K prefill: 114 flop/B is below the int8 and fp16 MFMA ridge",
                           "achieved_tflops": pre["layer_tflops"], "int8_peak_tops": INT8_PEAK_TOPS,
                           "frac_int8_peak": pre["layer_tflops"] / INT8_PEAK_TOPS,
                           "achieved_gbs": pre["layer_hbm_gbs"], "hbm_peak_gbs": HBM_PEAK_GBS,
                           "frac_hbm": pre["layer_hbm_gbs"] / HBM_PEAK_GBS}
    s235 = None
    if not a.no_stack235:
        s235 = stack235_leg(torch, L, a.stack235_layers, a.pool_gib, max(5, a.steps // 2), 2, a.stream_tokens)
        log(f"[bench] 235B stack: {json.dumps(s235)}")
    m30 = None
    if not a.no_model30b:
        m30 = model30b_leg(torch, L, a.model30b_layers, a.context, max(5, a.steps // 5), 2,
                                            tuple(int(t) for t in a.model30b_tokens.split(",")))
    cpu = None if a.no_cpu else cpu_baseline(a.tokens, a.cpu_seconds)
    gu_avg_s = main_res["stage_avg_us"]["gate_up"] * 1e-6
    achieved = main_res["gate_up_bytes"] / gu_avg_s / 1e9
    line = {
        "metric": "MoE FFN tok/s + % of HBM roofline (decode) / MFMA peak (prefill), 30B-A3B",
        "value": main_res["tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": main_res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"Qwen3-30B-A3B MoE FFN x {a.layers} layers, decode T={a.tokens}, Q8_0 experts, "
                               f"F16 router", "n_layer": a.layers, "tokens": a.tokens, "n_embd": H, "n_ff_exp": F,
                   "n_expert": E, "top_k": K, "expert_type": "Q8_0", "hip_graph": main_res["graph"]},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": measured_traffic("gate_up_T1") if (a.tokens == 1 and a.layers == N_LAYER) else None,
                     "traffic_source": "not measured in this run: FETCH_SIZE + WRITE_SIZE per gate_up launch from two "
                                       "rocprofv3 --pmc passes over this same command, scaled by a plain copy, kept in "
                                       "profiles/moe_decode_30b_q8_0_traffic.txt",
                     "kernel": "gate_up",
                     "kernel_avg_us": main_res["stage_avg_us"]["gate_up"],
                     "bytes_per_launch": main_res["gate_up_bytes"]},
        "stack_gbs": main_res["layer_gbs"],
        "ms_per_step_p10_p50_p90": main_res["ms_per_step_p10_p50_p90"],
        "stage_avg_us": main_res["stage_avg_us"],
        "t8": None if extra is None else {"tok_s": extra["tok_s"], "ms_per_step": extra["ms_per_step"],
                                          "ms_per_step_p10_p50_p90": extra["ms_per_step_p10_p50_p90"],
                                          "stack_gbs": extra["layer_gbs"], "stage_avg_us": extra["stage_avg_us"],
                                          "distinct_experts_per_layer": extra["distinct_experts_per_layer"]},
        "prefill": pre,
        "stack235": s235,
        "model30b": m30,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
