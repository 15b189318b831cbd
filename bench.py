"""MoE-layer throughput on one MI355X (BASELINE.json metric).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2]

Default workload: config 2 (the metric's decode configuration): 1000
independent single-token layer calls (T=1, d=640, E=128, k=4, I=640, f32
activations, int8 weights with per-channel scales). One step = the 1000
calls, enqueued as moe_layer_batched launches of W calls each (default: all
1000 in one) and replayed from a HIP graph. Every call has its own copy of
the layer's weights (158 MB each), so no call can reuse another's expert
bytes from L2 or the 256 MB MALL: each token's experts really stream from
HBM. The launch-bound figure — the same 1000 calls one at a time — is
reported beside it as sequential_tokens_per_s. Inputs are resident in HBM
before the timed region. Prints one JSON line.
"""
import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import runntime_amd as rt  # noqa: E402
from runntime_amd import perf  # noqa: E402
from runntime_amd.synth import CONFIGS, make_inputs, make_weight_copies  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def say(msg):
    print(msg, file=sys.stderr, flush=True)


def layer_bytes(cfg, n_experts_active):
    """Algorithmic HBM bytes of one layer call: the int8 weights and f32
    scales of the active experts, the f32 router weight, x in and out."""
    xb = 2 if cfg.x_dtype == "f16" else 4
    per_expert = 3 * cfg.d * cfg.I + 2 * cfg.I * 4 + cfg.d * 4
    return (n_experts_active * per_expert + cfg.d * cfg.E * 4 + cfg.T * cfg.d * (xb + 4))


def up_kernel_bytes(cfg, n_experts_active):
    """Algorithmic bytes of one gate/up launch: glu+lin int8 weights and
    scales of the active experts, the x rows it reads, the act rows it
    writes."""
    xb = 2 if cfg.x_dtype == "f16" else 4
    return (n_experts_active * (2 * cfg.d * cfg.I + 2 * cfg.I * 4)
            + cfg.T * cfg.d * xb + cfg.T * cfg.k * cfg.I * 4)


def layer_flops(cfg):
    return 2 * cfg.T * cfg.d * cfg.E + cfg.T * cfg.k * 6 * cfg.d * cfg.I


# HBM traffic per launch of the roofline kernel, from the committed
# FETCH_SIZE / WRITE_SIZE counter passes (calibrated against a plain copy);
# valid for the default launch shape of each workload.
TRAFFIC_PROFILES = {2: "k_expert_skinny_up_c2_decode_traffic.md",
                    3: "k_expert_skinny_up_c3_batched_decode_traffic.md",
                    "3-sequential": "k_expert_skinny_up_c3_decode_traffic.md",
                    4: "k_gemm_up_direct_c4_prefill_traffic.md",
                    5: "k_gemm_up_direct_c5_prefill_traffic.md"}


def source_sha():
    """SHA-256 (first 12 hex digits) over the kernel sources, runntime_amd/csrc/
    *.hip, *.h and *.cpp in name order: the same hash heads every kernel
    profile under profiles/, so a bench line and a profile of the same kernels
    can be matched."""
    import hashlib
    csrc = os.path.join(ROOT, "runntime_amd", "csrc")
    h = hashlib.sha256()
    for name in sorted(os.listdir(csrc)):
        if name.endswith((".hip", ".h", ".cpp")):
            h.update(name.encode())
            with open(os.path.join(csrc, name), "rb") as fh:
                h.update(fh.read())
    return h.hexdigest()[:12]


def profiled_traffic(config, default_shape):
    name = TRAFFIC_PROFILES.get(config)
    path = os.path.join(ROOT, "profiles", name) if name else None
    if not default_shape or path is None or not os.path.exists(path):
        return None, None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1]), "profiles/" + name
    return None, None


def cpu_baseline(cfg, seconds_budget=15.0):
    """The oracle's f32 restatement of the reference's WGSL kernels
    (topkSelect, moeUp, moeDown; router in the canonical f32 order), timed
    on this host's cores on a bounded sample of the same workload."""
    from oracle import ref
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or min(16, os.cpu_count() or 1)
    os.environ["OMP_NUM_THREADS"] = str(threads)
    inp = make_inputs(cfg, seed=1234, device="cpu", keep_q=True, T=64 if cfg.T == 1 else cfg.T)
    x = inp.x.float().numpy()
    pk = {n: (ref.pack_ekn(inp.q[n].numpy(), 8), getattr(inp, n).scales.numpy(),
              getattr(inp, n).bias.numpy()) for n in ("glu", "lin", "down")}
    rw, rb = inp.router_w.numpy(), inp.router_b.numpy()
    tokens = 0
    t0 = time.perf_counter()
    # single-token calls for the decode config, as the GPU runs them
    step_T = 1 if cfg.T == 1 else min(cfg.T, 64)
    i = 0
    while time.perf_counter() - t0 < seconds_budget:
        xs = x[i % len(x):i % len(x) + step_T] if step_T == 1 else x[:step_T]
        route = ref.topk(ref.router_logits(xs, rw, rb), cfg.k)
        act = ref.moe_up(xs, route, pk["glu"], pk["lin"], 8, cfg.d, cfg.E, f32ref=True)
        ref.moe_down(act, route, pk["down"], None, 8, cfg.I, cfg.E, f32ref=True)
        tokens += step_T
        i += 1
    dt = time.perf_counter() - t0
    return {"value": tokens / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
            "label": "restatement of the reference kernels, not the reference (the reference's "
                     "WGSL path needs Node >= 22, TypeGPU and Dawn, none of which this image has)",
            "sample": f"{tokens} tokens of {cfg.name} in {step_T}-token calls, {dt:.1f} s; "
                      "oracle/moe_oracle.c f32 restatement of topkSelect/moeUp/moeDown "
                      "(32-lane K split, fixed tree merge), OpenMP over rows"}


def bench_decode(cfg, args):
    """config 2: 1000 independent single-token calls per step. Each launch of
    moe_layer_batched runs W of them; call j uses weight copy j mod W, so no
    two calls in flight share a byte of weights and every copy is read again
    only after W·158 MB of other traffic (the 256 MB MALL cannot hold it)."""
    n_tok = cfg.tokens
    W = args.calls_per_launch
    say(f"drawing {W} weight copies of {cfg.name} on the GPU")
    wc = make_weight_copies(cfg, W, seed=100, device="cuda")
    g = torch.Generator().manual_seed(7)
    x = torch.randn((n_tok, 1, cfg.d), generator=g).to("cuda")
    residual = torch.zeros((n_tok, 1, cfg.d), dtype=torch.float32, device="cuda")
    out = torch.empty((n_tok, 1, cfg.d), dtype=torch.float32, device="cuda")
    routes = torch.empty((n_tok, 1, 2 * cfg.k), dtype=torch.float32, device="cuda")
    perf.reserve_batched(W, 1, cfg.d, cfg.I, cfg.E, cfg.k)

    def step():
        for j0 in range(0, n_tok, W):
            n = min(W, n_tok - j0)
            rt.moe_layer_batched(
                x[j0:j0 + n], wc.router_w[:n], wc.router_b[:n],
                rt.QuantExpertWeight(rt.QuantW(wc.glu.w.words[:n], wc.glu.w.dims), wc.glu.scales[:n], wc.glu.bias[:n]),
                rt.QuantExpertWeight(rt.QuantW(wc.lin.w.words[:n], wc.lin.w.dims), wc.lin.scales[:n], wc.lin.bias[:n]),
                rt.QuantExpertWeight(rt.QuantW(wc.down.w.words[:n], wc.down.w.dims), wc.down.scales[:n], wc.down.bias[:n]),
                residual[j0:j0 + n], cfg.k, out=out[j0:j0 + n], route=routes[j0:j0 + n])

    return step, n_tok


def bench_small_batched(cfg, args):
    """config 3 (default 16 calls; --c3-calls 0 runs them one at a time): N
    independent T-token calls per step, one moe_layer_batched launch, call c
    on weight copy c (no weights shared, so every call streams its own
    active experts' bytes). The same method as config 2's batched calls."""
    N = args.c3_calls
    say(f"drawing {N} weight copies of {cfg.name} on the GPU")
    wc = make_weight_copies(cfg, N, seed=400, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(9)
    xdt = torch.float16 if cfg.x_dtype == "f16" else torch.float32
    x = torch.randn((N, cfg.T, cfg.d), generator=g, device="cuda").to(xdt)
    residual = torch.zeros((N, cfg.T, cfg.d), dtype=torch.float32, device="cuda")
    out = torch.empty((N, cfg.T, cfg.d), dtype=torch.float32, device="cuda")
    routes = torch.empty((N, cfg.T, 2 * cfg.k), dtype=torch.float32, device="cuda")
    perf.reserve_batched(N, cfg.T, cfg.d, cfg.I, cfg.E, cfg.k)

    def step():
        rt.moe_layer_batched(x, wc.router_w, wc.router_b, wc.glu, wc.lin, wc.down, residual,
                             cfg.k, out=out, route=routes)

    def active():
        step()
        torch.cuda.synchronize()
        ids = routes[:, :, :cfg.k].long()
        return sum(int(torch.unique(ids[c]).numel()) for c in range(N)) / N

    return step, N * cfg.T, active


def sequential_rate(cfg, args):
    """The launch-bound case: the 1000 calls one at a time (W = 1), replayed
    from a graph. Reported beside the main figure."""
    wc = make_weight_copies(cfg, 4, seed=300, device="cuda")
    g = torch.Generator().manual_seed(9)
    n_tok = cfg.tokens
    x = torch.randn((n_tok, 1, cfg.d), generator=g).to("cuda")
    out = torch.empty((n_tok, 1, cfg.d), dtype=torch.float32, device="cuda")
    routes = torch.empty((n_tok, 1, 2 * cfg.k), dtype=torch.float32, device="cuda")
    perf.reserve_batched(1, 1, cfg.d, cfg.I, cfg.E, cfg.k)

    def step():
        for j in range(n_tok):
            c = j % 4
            rt.moe_layer_batched(
                x[j:j + 1], wc.router_w[c:c + 1], wc.router_b[c:c + 1],
                rt.QuantExpertWeight(rt.QuantW(wc.glu.w.words[c:c + 1], wc.glu.w.dims), wc.glu.scales[c:c + 1], wc.glu.bias[c:c + 1]),
                rt.QuantExpertWeight(rt.QuantW(wc.lin.w.words[c:c + 1], wc.lin.w.dims), wc.lin.scales[c:c + 1], wc.lin.bias[c:c + 1]),
                rt.QuantExpertWeight(rt.QuantW(wc.down.w.words[c:c + 1], wc.down.w.dims), wc.down.scales[c:c + 1], wc.down.bias[c:c + 1]),
                None, cfg.k, out=out[j:j + 1], route=routes[j:j + 1])

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        step()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            step()
        graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / 3
    del wc, graph
    torch.cuda.empty_cache()
    return n_tok / dt


def copy_calibration(mib):
    """4 launches of a plain copy of `mib` MiB (torch's copy kernel): under
    rocprofv3 --pmc FETCH_SIZE (or WRITE_SIZE) each dispatch moves exactly
    mib MiB each way, which converts the counter's reading to bytes."""
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_per_launch": n * 4, "launches": 4}), flush=True)


def gemm_calibration(config):
    """The vendor library's dense f16 GEMM (torch.matmul → hipBLASLt) at the
    grouped GEMMs' shapes with every expert's rows stacked: M = T·k, N and K
    of the up (N = 2·I: glu and lin) and down products. It has no int8
    conversion, gather, grouping or padding: a practical ceiling for f16 MFMA
    work of that size on this GPU, reported beside the 2.5 PF peak."""
    cfg = CONFIGS[config]
    M = cfg.T * cfg.k
    res = {}
    for name, n, k in (("up", 2 * cfg.I, cfg.d), ("down", cfg.d, cfg.I)):
        a = torch.randn(M, k, device="cuda", dtype=torch.float16)
        b = torch.randn(k, n, device="cuda", dtype=torch.float16)
        for _ in range(3):
            a @ b
        torch.cuda.synchronize()
        reps = 20
        t0 = time.perf_counter()
        for _ in range(reps):
            a @ b
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / reps
        res[name] = {"M": M, "N": n, "K": k, "ms": round(dt * 1e3, 4),
                     "tflops": round(2 * M * n * k / dt / 1e12, 1),
                     "frac_of_peak": round(2 * M * n * k / dt / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
    print(json.dumps({"gemm_calibration": cfg.name, "dense_f16_torch_matmul": res}), flush=True)


def float_block_bench(args):
    """The float-weight block (moe_block_float) at config 2's layer shape
    (d = I = 640, E = 128, k = 4) with f16 or f32 expert weights and
    `--float-tokens` tokens per call: one line with tokens/s and the
    expert-weight stream rate (the distinct active experts' glu, lin and out
    weights per call, over the measured time of the gate/up and down
    launches)."""
    cfg = CONFIGS[2]
    dt = torch.float16 if args.float == "f16" else torch.float32
    T, d, I, E, k = args.float_tokens, cfg.d, cfg.I, cfg.E, cfg.k
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn((T, d), generator=g, device="cuda").to(dt)
    norm = (1 + 0.1 * torch.randn(d, generator=g, device="cuda")).to(dt)
    rw = 0.02 * torch.randn((d, E), generator=g, device="cuda")
    mk = lambda r, c, s: (s * torch.randn((r, c), generator=g, device="cuda")).to(dt)
    glu, lin, down = mk(E * d, I, d ** -0.5), mk(E * d, I, d ** -0.5), mk(E * I, d, I ** -0.5)
    gb, lb, db = mk(E, I, 0.1), mk(E, I, 0.1), mk(E, d, 0.1)

    def step():
        return rt.moe_block_float(x, norm, 1e-5, rw, None, glu, gb, lin, lb, down, db, k=k)

    for _ in range(max(1, args.warmup)):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt_s = (time.perf_counter() - t0) / args.steps
    perf.read(reset=True)
    perf.enable(True)
    out, route = rt.moe_block_float(x, norm, 1e-5, rw, None, glu, gb, lin, lb, down, db, k=k,
                                    return_route=True)
    torch.cuda.synchronize()
    groups = perf.read(reset=True)
    perf.enable(False)
    active = int(torch.unique(route[:, :k]).numel())
    esize = 2 if dt == torch.float16 else 4
    wbytes = active * 3 * d * I * esize
    up_ms = groups.get("up", (0.0, 1))[0] / max(groups.get("up", (0.0, 1))[1], 1)
    dn_ms = groups.get("down", (0.0, 1))[0] / max(groups.get("down", (0.0, 1))[1], 1)
    gbs = wbytes / ((up_ms + dn_ms) / 1e3) / 1e9
    print(json.dumps({
        "metric": "float-weight MoE block tokens/s at 1 MI355X", "value": round(T / dt_s, 1),
        "unit": "tokens/s", "ms_per_step": round(dt_s * 1e3, 4), "dtype": args.float,
        "config": {"workload": f"float_block_T{T}_d{d}_E{E}_k{k}_I{I}_{args.float}",
                   "active_experts": active},
        "kernel_ms": {kk: round(v[0] / max(v[1], 1), 5) for kk, v in groups.items()},
        "expert_stream": {"bytes": wbytes, "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}}), flush=True)


def privacy_filter_bench(args):
    """The whole privacy-filter network (8 blocks of attention + the int8
    MoE block, E = 128, k = 4, d = I = 640, 33 classes) with random int8
    weights, text in token ids to labelled spans out: embedding gather,
    forward on the GPU, logits to the host, log-softmax, constrained Viterbi,
    spans. --pf-texts texts with lengths drawn from 12..100 tokens (the
    reference's 300 messages of 9-76 words), one text per call; the line
    reports the median ms per text (the reference's figure: 16.4 ms on an
    Apple M2 Pro over WebGPU, tokenizer included; none runs here)."""
    import numpy as np
    from runntime_amd import privacy_filter as pf
    from runntime_amd.checkpoint import MoeBlock
    from runntime_amd.linear import Linear
    from runntime_amd.quantw import QuantExpertWeight, QuantW
    rng = np.random.default_rng(0)
    dev = "cuda"
    E, k, d, I, vocab = 128, 4, 640, 640, 200064
    g = torch.Generator(device=dev).manual_seed(1)

    def qlin(out_f, in_f, gs, bias=True):
        ints = rng.integers(-127, 128, size=(out_f, in_f)).astype(np.int8)
        sc = (rng.uniform(0.5, 1.5, size=(out_f, in_f // gs)) / (127 * np.sqrt(in_f))).astype(np.float32)
        return Linear.from_quant(ints, sc, 8, rng.standard_normal(out_f).astype(np.float32) * 0.1
                                 if bias else None, dev)

    def expert(K, N):
        q = torch.randint(-127, 128, (E, K, N), generator=g, device=dev, dtype=torch.int8)
        words = rt.pack_expert_weights_torch(q)
        return QuantExpertWeight(QuantW(words, (E * K, N)),
                                 0.5e-3 + 1.5e-3 * torch.rand((E, N), generator=g, device=dev),
                                 0.01 * torch.randn((E, N), generator=g, device=dev))

    say("building the model (8 blocks, random int8 weights)")
    blocks = []
    for _ in range(8):
        attn = pf.AttnBlock(torch.ones(d, device=dev), qlin(1152, 640, 640), qlin(640, 896, 128),
                            torch.randn(14, generator=g, device=dev))
        mlp = MoeBlock(norm_w=torch.ones(d, device=dev),
                       router_w=0.02 * torch.randn((d, E), generator=g, device=dev), router_b=None,
                       glu=expert(d, I), lin=expert(d, I), down=expert(I, d), E=E, d=d, I=I,
                       bits=8, group_up=d, group_down=I, k=k)
        blocks.append(pf.Block(attn, mlp))
    emb = rng.standard_normal((vocab, d), dtype=np.float32)
    model = pf.PrivacyFilterModel(emb, blocks, torch.ones(d, device=dev), qlin(36, 640, 640, False))
    info = pf.build_label_info(pf.V2_NER_CLASS_NAMES)
    dec = pf.ViterbiDecoder(info)
    lengths = rng.integers(12, 101, size=args.pf_texts)
    texts = [rng.integers(0, vocab, size=n) for n in lengths]

    fwd = model.forward
    if not args.no_graph:
        say(f"capturing the forward for {len(set(lengths.tolist()))} text lengths")
        fwd = pf.GraphedForward(model, lengths.tolist())

    def detect(ids):
        logits = fwd(ids)[:, :33].cpu().numpy()
        return pf.labels_to_spans(dec.decode(pf.log_softmax_rows(logits)), info)

    for ids in texts[:max(1, args.warmup)]:
        detect(ids)
    torch.cuda.synchronize()
    times = []
    t_all = time.perf_counter()
    for ids in texts:
        t0 = time.perf_counter()
        detect(ids)
        times.append(time.perf_counter() - t0)
    total = time.perf_counter() - t_all
    med = float(np.median(times)) * 1e3
    print(json.dumps({
        "metric": "privacy filter ms per text (median) at 1 MI355X", "value": round(med, 3),
        "unit": "ms", "higher_is_better": False, "texts": len(texts),
        "texts_per_s": round(len(texts) / total, 1), "dtype": "int8 weights, f32 activations",
        "data": "synthetic (random int8 weights of the model's shapes, random token ids)",
        "config": {"workload": "privacy_filter_8blocks_E128_k4_d640_I640",
                   "tokens_per_text": [int(lengths.min()), int(lengths.max())],
                   "median_tokens": int(np.median(lengths)), "graph": not args.no_graph},
        "reference_published": {"value": 16.4, "unit": "ms per text (median)",
                                "hardware": "Apple M2 Pro, WebGPU/Metal, tokenizer included"}}),
        flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--copies", type=int, default=2, help="rotating input sets (config 3)")
    ap.add_argument("--c3-calls", type=int, default=16,
                    help="config 3: N independent calls (own weight copies) per batched launch; "
                         "0 runs --copies calls one at a time")
    ap.add_argument("--calls-per-launch", type=int, default=1000,
                    help="config 2: independent single-token calls per batched launch")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-sequential", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MiB",
                    help="only run 4 plain device copies of MiB each (reference reading "
                         "for the FETCH_SIZE / WRITE_SIZE counters) and exit")
    ap.add_argument("--float", choices=["f16", "f32"], default=None,
                    help="only time the float-weight block (moe_block_float) at config 2's "
                         "layer shape and exit")
    ap.add_argument("--float-tokens", type=int, default=32)
    ap.add_argument("--privacy-filter", action="store_true",
                    help="only time the whole privacy-filter network, text (token ids) to spans, "
                         "per text, and exit")
    ap.add_argument("--pf-texts", type=int, default=300)
    ap.add_argument("--gemm-calibration", action="store_true",
                    help="only time torch.matmul (hipBLASLt) dense f16 GEMMs of the config's "
                         "up/down shapes and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)
    torch.cuda.set_device(0)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gemm_calibration:
        gemm_calibration(args.config)
        return
    if args.float:
        float_block_bench(args)
        return
    if args.privacy_filter:
        privacy_filter_bench(args)
        return
    cfg = CONFIGS[args.config]

    c3_active = None
    if args.config == 2:
        step, tokens_per_step = bench_decode(cfg, args)
    elif args.config == 3 and args.c3_calls > 0:
        step, tokens_per_step, c3_active = bench_small_batched(cfg, args)
    else:
        C = args.copies if args.config == 3 else 1
        say(f"building {C} input set(s) of {cfg.name}")
        sets = [make_inputs(cfg, seed=200 + c, device="cuda") for c in range(C)]
        out = torch.empty((cfg.T, cfg.d), dtype=torch.float32, device="cuda")
        route = torch.empty((cfg.T, 2 * cfg.k), dtype=torch.float32, device="cuda")
        perf.reserve(cfg.T, cfg.d, cfg.I, cfg.E, cfg.k)
        counter = [0]

        def step():
            for c in range(C):
                w = sets[c]
                rt.moe_layer(w.x, w.router_w, w.router_b, w.glu, w.lin, w.down, w.residual,
                             cfg.k, out=out, route=route)
        tokens_per_step = cfg.T * C

    stream = torch.cuda.Stream()
    graph = None
    with torch.cuda.stream(stream):
        for _ in range(max(1, args.warmup)):
            step()
        torch.cuda.synchronize()
        if not args.no_graph:
            say("capturing graph")
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                step()
            torch.cuda.synchronize()
            for _ in range(args.warmup):
                graph.replay()
        torch.cuda.synchronize()

        say(f"timing {args.steps} steps")
        t0 = time.perf_counter()
        for _ in range(args.steps):
            if graph is not None:
                graph.replay()
            else:
                step()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0

        # Per-kernel durations: one more eager step with the event sink on.
        perf.read(reset=True)
        perf.enable(True)
        step()
        torch.cuda.synchronize()
        groups = perf.read(reset=True)
        perf.enable(False)

    ms_per_step = elapsed * 1e3 / args.steps
    value = tokens_per_step * args.steps / elapsed

    # Experts touched per call: a single token routes to k distinct experts;
    # for more tokens, the distinct ids of each input set's actual route
    # (the same router as the layer's), averaged over the sets.
    if args.config == 2:
        active_per_call = cfg.k
        calls = tokens_per_step
        W = args.calls_per_launch
    elif c3_active is not None:
        active_per_call = c3_active()
        calls = tokens_per_step // cfg.T
        W = args.c3_calls
    else:
        W = 1
        counts = []
        for w in sets:
            r = rt.router_topk(w.x, w.router_w, w.router_b, cfg.k)
            counts.append(int(torch.unique(r[:, :cfg.k]).numel()))
        active_per_call = sum(counts) / len(counts)
        calls = tokens_per_step // cfg.T
    up_ms, up_n = groups.get("up", (0.0, 0))
    up_avg_s = up_ms / max(up_n, 1) / 1e3
    default_shape = ((args.config == 2 and args.calls_per_launch == 1000)
                     or (args.config == 3 and args.c3_calls in (0, 16) and args.copies == 2)
                     or args.config in (4, 5))
    traffic, traffic_src = profiled_traffic(
        "3-sequential" if args.config == 3 and args.c3_calls == 0 else args.config, default_shape)
    if args.config in (2, 3):
        per_launch = round(up_kernel_bytes(cfg, active_per_call) * W)
        achieved = per_launch / up_avg_s / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                    "traffic_source": traffic_src,
                    "kernel": "k_expert_skinny<up> (gate/up + SwiGLU)",
                    "algorithmic_bytes_per_launch": per_launch,
                    "active_experts_per_call": active_per_call,
                    "avg_launch_us": round(up_avg_s * 1e6, 2)}
        layer_frac = layer_bytes(cfg, active_per_call) * calls / (ms_per_step / 1e3) / 1e9 / HBM_PEAK_GBS
    else:
        fl = cfg.T * cfg.k * 4 * cfg.d * cfg.I
        achieved = fl / up_avg_s / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_F16_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4),
                    "traffic": traffic, "traffic_source": traffic_src,
                    "kernel": "k_gemm_up_direct (gate/up grouped GEMM + SwiGLU)",
                    "algorithmic_flops_per_launch": fl, "avg_launch_us": round(up_avg_s * 1e6, 2)}
        layer_frac = layer_flops(cfg) * calls / (ms_per_step / 1e3) / 1e12 / MFMA_F16_PEAK_TFLOPS
        # The down product (k_gemm_down_i8: three int8 MFMAs per product on
        # act's int8 limbs), against the same f16 peak in algorithmic flops.
        dn_ms, dn_n = groups.get("down", (0.0, 0))
        dn_fl = cfg.T * cfg.k * 2 * cfg.d * cfg.I
        dn_avg_s = dn_ms / max(dn_n, 1) / 1e3
        roofline["down"] = {"kernel": "k_gemm_down_i8 (down grouped GEMM, int8 MFMA on act limbs)",
                            "algorithmic_flops_per_launch": dn_fl,
                            "avg_launch_us": round(dn_avg_s * 1e6, 2),
                            "achieved": round(dn_fl / dn_avg_s / 1e12, 2),
                            "frac": round(dn_fl / dn_avg_s / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}

    rows = None
    if args.config in (4, 5):
        r = rt.router_topk(sets[0].x, sets[0].router_w, sets[0].router_b, cfg.k)
        cnt = torch.bincount(r[:, :cfg.k].reshape(-1).long(), minlength=cfg.E)
        rows = {"min": int(cnt.min()), "max": int(cnt.max()),
                "experts_without_rows": int((cnt == 0).sum()),
                "hottest_share_of_tokens": round(int(cnt.max()) / cfg.T, 4)}
    line = {
        "metric": "MoE-layer tokens/s at 1 MI355X",
        "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded; int8 weights U[-127,127], scales U(0.5e-3,2e-3), x~N(0,1))",
        "config": {"workload": cfg.name, "T": cfg.T, "d": cfg.d, "E": cfg.E, "k": cfg.k,
                   "I": cfg.I, "x_dtype": cfg.x_dtype, "tokens_per_step": tokens_per_step,
                   "calls_per_step": calls,
                   "calls_per_launch": W if args.config in (2, 3) else 1,
                   "weight_copies": (args.calls_per_launch if args.config == 2
                                     else (args.c3_calls or args.copies) if args.config == 3
                                     else 1),
                   "graph": graph is not None, "parallelism": "single GPU",
                   "arith": ("int8 weights exact in f16 MFMA, f32 accumulate; act between the "
                             "prefill products as 24-bit fixed point in three int8 limbs on "
                             "int8 MFMA, i32 accumulate" if args.config in (4, 5) else
                             "int8 weights exact in f16 MFMA, f32 inputs split hi+lo, "
                             "f32 accumulate")},
        "layer_roofline_frac": round(layer_frac, 4),
        **({"rows_per_expert": rows} if rows else {}),
        "kernel_ms": {g: round(ms / n, 5) for g, (ms, n) in groups.items()},
        "roofline": roofline,
        "source_sha": source_sha(),
    }
    if args.config == 2 and not args.no_sequential:
        say("sequential (launch-bound) rate")
        line["sequential_tokens_per_s"] = round(sequential_rate(cfg, args), 1)
    if not args.no_cpu_baseline:
        say("cpu baseline")
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
