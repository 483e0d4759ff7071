"""Headline benchmark: bs=1 self-speculative decode on one MI355X.

Workload: the 16-layer, 1536-hidden GLM decoder (16 q / 2 kv heads, head_dim 128, SwiGLU 4608, vocab 59392, bf16,
random N(0, 0.02) weights, seed 2); prompt = 2048 visual embeddings N(0,1) + 6144 text ids U[0, vocab) (the first
32 are the prompt, the rest fill the KV prefix to 8K), prefilled (untimed) into 16-token pages; then full-draft rounds
with B = 16 (K = 17 rows per forward: draft forward + verify forward + argmax/accept/bonus + KV commit) until 512
tokens are committed. A "step" is one round. Each round is one HIP-graph replay; lengths live on the device.

Reported next to it, in the same JSON line:
  * AR decode of the same model on the same GPU (one 1-row forward per token, also graph-replayed);
  * planted-acceptance rounds: the draft is overwritten with the AR tokens up to a mismatch ~ geometric(0.1)
    (capped at B), so the verify accepts what a trained draft would (kernel cost per round does not depend on it);
  * roofline of the block-diffusion draft attention at the round's shape (HIP events on its stream), timed over 48
    distinct caches so its K/V comes from HBM (`--attn-only` runs just this measurement, for rocprof);
  * the CPU baseline: the oracle's full-draft round (fp32 torch) on the host cores, from the same 8K state.

    python bench.py [--steps K] [--warmup W] [--no-cpu] [--prefix 8192] [--tokens 512] [--bd 16]
"""
import argparse
import json
import os
import sys
import time

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def cpu_info():
    """The host's CPU model and its physical cores and logical threads (lscpu's fields, read from /proc/cpuinfo)."""
    model, cores = None, set()
    try:
        phys = core = None
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    cores.add((phys, core))
        if phys is not None:
            cores.add((phys, core))
    except OSError:
        pass
    return {"cpu_model": model, "physical_cores": len(cores) or None, "logical_threads": os.cpu_count(),
            "torch_threads": torch.get_num_threads()}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def attn_bytes(L, W, Hq=16, Hkv=2, D=128):
    """algorithmic HBM bytes of one window-attention call: K and V of L+W tokens + Q and O of W rows (bf16)."""
    return 2 * Hkv * D * 2 * (L + W) + 2 * W * Hq * D * 2


def attn_flops(L, W, Hq=16, D=128):
    return 4 * W * Hq * D * (L + W)


ATTN_COPIES = 48  # distinct KV caches the attention timing cycles through (48 x 8.7 MB > the 256 MB Infinity Cache)
COPY_BYTES = 64 << 20  # the plain copy whose HBM counters calibrate FETCH_SIZE / WRITE_SIZE


def attn_roofline(dev, L, W, cap, n_causal=1, copies=ATTN_COPIES, Hq=16, Hkv=2, D=128):
    """Average duration of one draft (n_causal=1) or verify (None) attention call (gss_draft_attn / gss_verify_attn:
    split kernel + merge) at prefix L, window W, capacity cap, over ``copies`` distinct random caches in shuffled
    16-token pages, so the K/V stream comes from HBM as in a round. Returns microseconds per call."""
    from gravityocr_amd import kernels as K
    g = torch.Generator(device=dev).manual_seed(1)
    pages = (cap + 15) // 16
    kp = torch.randn(copies, pages, Hkv, 16, D, device=dev, generator=g).div_(D ** 0.5).bfloat16()
    vp = torch.randn(copies, pages, Hkv, D, 16, device=dev, generator=g).div_(D ** 0.5).bfloat16()
    pt = torch.randperm(pages, device=dev, generator=g).int().view(1, -1)
    q = torch.randn(1, W, Hq, D, device=dev, generator=g).div_(D ** 0.5).bfloat16()
    kw = torch.randn(1, W, Hkv, D, device=dev, generator=g).div_(D ** 0.5).bfloat16()
    vw = torch.randn_like(kw)
    o = torch.empty_like(q)
    sl = torch.tensor([L], dtype=torch.int32, device=dev)
    ws = torch.zeros(max(1, K.attn_workspace_bytes(1, Hq, Hkv, D, W, cap)), dtype=torch.uint8, device=dev)
    fns = [lambda i=i: K.window_attention(q, kp[i], vp[i], pt, sl, kw, vw, o, n_causal=n_causal, scale=D ** -0.5,
                                          max_kv_len=cap, workspace=ws) for i in range(copies)]
    return time_kernel(fns, n=2)


def attn_batched_roofline(dev, W=17, bs=32, copies=2, Hq=16, Hkv=2, D=128, seed=3):
    """The batched draft attention (bs sequences, prefixes L_i ~ U[1024, 12288] with a seeded generator, one shared
    pool of 16-token pages in shuffled order, window W): average call duration over ``copies`` distinct pools (each
    ~0.4 GB, together more than the Infinity Cache). Returns (microseconds per call, algorithmic bytes per call,
    flops of the two contractions per call)."""
    from gravityocr_amd import kernels as K
    Ls = np.random.default_rng(seed).integers(1024, 12289, size=bs)
    cap = int(Ls.max()) + W + 64
    ppseq = (cap + 15) // 16
    g = torch.Generator(device=dev).manual_seed(seed)
    n_pages = bs * ppseq
    pools = []
    for _ in range(copies):
        kp = torch.empty(n_pages, Hkv, 16, D, dtype=torch.bfloat16, device=dev).normal_(0, D ** -0.5, generator=g)
        vp = torch.empty(n_pages, Hkv, D, 16, dtype=torch.bfloat16, device=dev).normal_(0, D ** -0.5, generator=g)
        pools.append((kp, vp))
    pt = torch.randperm(n_pages, device=dev, generator=g).int().view(bs, ppseq)
    q = torch.randn(bs, W, Hq, D, device=dev, generator=g).div_(D ** 0.5).bfloat16()
    kw = torch.randn(bs, W, Hkv, D, device=dev, generator=g).div_(D ** 0.5).bfloat16()
    vw = torch.randn_like(kw)
    o = torch.empty_like(q)
    sl = torch.tensor(Ls, dtype=torch.int32, device=dev)
    ws = torch.zeros(max(1, K.attn_workspace_bytes(bs, Hq, Hkv, D, W, cap)), dtype=torch.uint8, device=dev)
    fns = [lambda kp=kp, vp=vp: K.window_attention(q, kp, vp, pt, sl, kw, vw, o, n_causal=1, scale=D ** -0.5,
                                                   max_kv_len=cap, workspace=ws) for kp, vp in pools]
    us = time_kernel(fns, n=4, reps=3)
    nbytes = sum(2 * Hkv * D * 2 * (int(L) + W) for L in Ls) + 2 * bs * W * Hq * D * 2
    flops = sum(attn_flops(int(L), W, Hq, D) for L in Ls)
    return us, nbytes, flops


def argmax_roofline(dev, b, W=17, V=59392):
    """gss_argmax_accept at the accept shape: bf16 logits [b, W, V] (b * W * V * 2 bytes) with the window, accept,
    next boundary token and packed row outputs, cycled over enough distinct logits buffers (> 256 MB together) that
    they come from HBM. Returns (microseconds per call, algorithmic bytes per call)."""
    from gravityocr_amd import kernels as K
    nbytes = b * W * V * 2
    copies = max(2, -(-(320 << 20) // nbytes))
    g = torch.Generator(device=dev).manual_seed(11)
    lg = torch.randn(copies, b, W, V, device=dev, generator=g).bfloat16()
    win = torch.randint(0, V, (b, W), device=dev, generator=g, dtype=torch.int32)
    tgt = torch.empty(b, W, dtype=torch.int32, device=dev)
    acc, x0 = (torch.empty(b, dtype=torch.int32, device=dev) for _ in range(2))
    packed = torch.empty(b, W + 2, dtype=torch.int32, device=dev)
    ws = torch.zeros(K.argmax_workspace_bytes(b, W, V), dtype=torch.uint8, device=dev)
    fns = [lambda i=i: K.argmax_accept(lg[i], tgt, ws, window=win, accept_len=acc, next_x0=x0, packed=packed)
           for i in range(copies)]
    return time_kernel(fns, n=max(1, 256 // copies)), nbytes


def commit_roofline(dev, n_rows=17, L=8448, layers=16, Hkv=2, D=128, reps=5, n=64):
    """gss_kv_commit of a whole verify window at bs = 1 (the 16-layer decoder's staging, all n_rows rows kept) into
    16-token pages at prefix L. Algorithmic bytes: the rows read from the staging and written to the pages, K and V,
    every layer. The n calls of a timed graph append n windows (the length is reset between replays, outside the
    timed region). Returns (microseconds per call, algorithmic bytes per call)."""
    from gravityocr_amd import kernels as K
    cap = L + (n + 2) * n_rows + 64
    ppseq = (cap + 15) // 16
    g = torch.Generator(device=dev).manual_seed(12)
    kw = torch.randn(layers, 1, n_rows, Hkv, D, device=dev, generator=g).bfloat16()
    vw = torch.randn_like(kw)
    kp = torch.zeros(layers, ppseq, Hkv, 16, D, dtype=torch.bfloat16, device=dev)
    vp = torch.zeros(layers, ppseq, Hkv, D, 16, dtype=torch.bfloat16, device=dev)
    pt = torch.randperm(ppseq, device=dev, generator=g).int().view(1, -1)
    sl = torch.tensor([L], dtype=torch.int32, device=dev)
    ws = torch.zeros(K.commit_workspace_bytes(1), dtype=torch.uint8, device=dev)
    K.kv_commit(kw, vw, kp, vp, pt, sl, ws, n_add=n_rows)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    sl.fill_(L)
    with torch.cuda.graph(gr):
        for _ in range(n):
            K.kv_commit(kw, vw, kp, vp, pt, sl, ws, n_add=n_rows)
    total = 0.0
    for _ in range(reps):
        sl.fill_(L)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        gr.replay()
        e1.record()
        torch.cuda.synchronize()
        total += e0.elapsed_time(e1)
    return total * 1e3 / (reps * n), 2 * 2 * layers * n_rows * Hkv * D * 2


def batched_rounds(dev, w, cfg, block_sizes=(8, 16, 32), rounds=256, bs=32, seed=3):
    """The batched serving shape: bs sequences with prefixes L_i ~ U[1024, 12288] (seed 3) in one shuffled pool of
    16-token pages, prefix K/V seeded N(0, 0.8) (the spread of this model's projected K/V; the kernels' cost does not
    depend on the values), each sequence's x0 a seeded random id. For each block size: ``rounds`` graph-replayed
    full-draft rounds of the whole batch (every sequence its own accept length), and as many graph-replayed AR steps
    of the batch. Returns a dict per block size."""
    from gravityocr_amd.engine import GssEngine, SelfSpecDecoder
    rng = np.random.default_rng(seed)
    L0 = rng.integers(1024, 12289, size=bs)
    max_bd = max(block_sizes)
    eng = GssEngine(cfg, w, max_bs=bs, max_len=int(L0.max()) + rounds * (max_bd + 2) + 2 * (max_bd + 2) + 64,
                    device=dev, page_seed=seed, max_win=max_bd + 2)
    g = torch.Generator(device=dev).manual_seed(seed)
    eng.k_pages.normal_(0.0, 0.8, generator=g)
    eng.v_pages.normal_(0.0, 0.8, generator=g)
    x0 = torch.tensor(rng.integers(0, cfg.vocab - 1, size=bs), dtype=torch.int32, device=dev)
    L0_dev = torch.tensor(L0, dtype=torch.int32, device=dev)
    out = {}
    for bd in block_sizes:
        dec = SelfSpecDecoder(eng, bd=bd, mask_id=cfg.vocab - 1, bs=bs, max_rounds=rounds + 8)

        def reset():
            eng.seq_lens[:bs].copy_(L0_dev)
            dec.start(x0)

        reset()
        dec.round()
        reset()
        dec.ar_step()
        reset()
        dec.capture()
        reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(rounds):
            dec.g_round.replay()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        accs = dec.accept_lengths(rounds)                                   # [rounds, bs]
        n_commit = int((accs + 2).sum())
        reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(rounds):
            dec.g_ar.replay()
        torch.cuda.synchronize()
        adt = time.perf_counter() - t0
        per_seq = [np.bincount(accs[:, b], minlength=bd + 1).tolist() for b in range(bs)]
        out[str(bd)] = {"K": bd + 1, "rounds": rounds, "round_us": round(dt / rounds * 1e6, 1),
                        "committed_tokens": n_commit, "tokens_per_s": round(n_commit / dt, 1),
                        "ar_step_us": round(adt / rounds * 1e6, 1), "ar_tokens_per_s": round(bs * rounds / adt, 1),
                        "speedup_vs_ar": round((n_commit / dt) / (bs * rounds / adt), 3),
                        "mean_committed_per_round_per_seq": round(n_commit / (rounds * bs), 3),
                        "accept_hist": np.bincount(accs.reshape(-1), minlength=bd + 1).tolist(),
                        "accept_hist_per_seq": per_seq}
        log(f"batched B={bd}: {out[str(bd)]['round_us']} us/round, {out[str(bd)]['tokens_per_s']} tokens/s, "
            f"AR {out[str(bd)]['ar_tokens_per_s']} tokens/s")
        del dec
    out["prefixes"] = {"min": int(L0.min()), "max": int(L0.max()), "sum": int(L0.sum())}
    del eng
    torch.cuda.empty_cache()
    return out


def copy_calibration(dev, reps=3):
    """Plain device copies of COPY_BYTES, as an elementwise kernel (reads COPY_BYTES, writes COPY_BYTES): the
    calibration kernel of the FETCH_SIZE / WRITE_SIZE passes."""
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(reps):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()


def from_profile(name, key, cast=float):
    """A figure of a committed profile summary (profiles/<name>: lines `key: value`, written from rocprofv3 --pmc
    passes: HBM traffic per call from FETCH_SIZE / WRITE_SIZE scaled by the copy calibration, MFMA utilisation), or
    None when it is absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return cast(line.split(":")[1])
    except OSError:
        pass
    return None


def time_kernel(fn, n=100, reps=5):
    """average duration of one launch of fn (a callable, or a list of callables launched in turn): n passes captured
    back to back in one HIP graph (no host work between them), replayed ``reps`` times between HIP events on the
    capture/launch stream; returns microseconds."""
    fns = fn if isinstance(fn, (list, tuple)) else [fn]
    for f in fns:
        f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(n):
            for f in fns:
                f()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (n * reps * len(fns))  # us


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=0, help="timed rounds (0 = the rounds that commit --tokens)")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--prefix", type=int, default=8192)
    ap.add_argument("--tokens", type=int, default=512)
    ap.add_argument("--bd", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--profile-only", action="store_true", help="skip AR, planted and CPU legs (for rocprof runs)")
    ap.add_argument("--ar-only", action="store_true", help="only the graph-replayed AR steps (for rocprof runs)")
    ap.add_argument("--sampled-only", action="store_true", help="only the graph-replayed sampled rounds (for rocprof runs)")
    ap.add_argument("--attn-only", action="store_true",
                    help="only the draft-attention roofline measurement and the copy calibration (for rocprof runs)")
    ap.add_argument("--attn-batched-only", action="store_true",
                    help="only the batched (32 ragged sequences) draft-attention measurement (for rocprof runs)")
    ap.add_argument("--batched-only", action="store_true",
                    help="only the batched rounds (32 ragged sequences, B in 8/16/32) (for rocprof runs)")
    ap.add_argument("--no-batched", action="store_true", help="skip the batched rounds")
    ap.add_argument("--prefill-only", action="store_true", help="only the prefill, cold then warm (for rocprof runs)")
    ap.add_argument("--batched-rounds", type=int, default=256)
    ap.add_argument("--small-only", action="store_true",
                    help="only the argmax / accept and KV-commit measurements (for rocprof runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the self-spec round shards by sequence (no collective), so a multi-GPU "
              "figure is N independent copies of this one; run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.attn_only:
        dev = torch.device("cuda:0")
        L, Kw = args.prefix + args.tokens // 2, args.bd + 1
        cap = args.prefix + args.tokens + 4 * (Kw + 1) + 64
        d_us = attn_roofline(dev, L, Kw, cap)
        copy_calibration(dev)
        ab = attn_bytes(L, Kw)
        print(json.dumps({"kernel": "gss_draft_attn", "L": L, "W": Kw, "avg_us": round(d_us, 2),
                          "algorithmic_bytes": ab, "achieved_GBs": round(ab / (d_us * 1e-6) / 1e9, 1),
                          "copy_bytes": COPY_BYTES}), flush=True)
        return
    if args.attn_batched_only:
        b_us, b_bytes, _ = attn_batched_roofline(torch.device("cuda:0"), W=args.bd + 1)
        print(json.dumps({"kernel": "gss_draft_attn batched", "W": args.bd + 1, "avg_us": round(b_us, 2),
                          "algorithmic_bytes": b_bytes, "achieved_GBs": round(b_bytes / (b_us * 1e-6) / 1e9, 1)}),
              flush=True)
        return

    from gravityocr_amd.engine import GssEngine, SelfSpecDecoder
    from gravityocr_amd.model import SYNTH_1536 as cfg, synthetic_prompt, synthetic_weights
    from gravityocr_amd import kernels as K

    dev = torch.device("cuda:0")
    if args.small_only:
        res = {"argmax": {str(b): round(argmax_roofline(dev, b)[0], 2) for b in (1, 8, 32)},
               "kv_commit_us": round(commit_roofline(dev)[0], 2)}
        print(json.dumps(res), flush=True)
        return
    bd, Kw, P = args.bd, args.bd + 1, args.prefix
    t0 = time.time()
    w = synthetic_weights(cfg, seed=2)
    vis, ids = synthetic_prompt(cfg, 2048, P - 2048, seed=2)
    emb = torch.cat([vis, w["embed"][ids]], 0)
    log(f"weights + prompt drawn in {time.time() - t0:.1f}s")
    if args.batched_only:
        print(json.dumps(batched_rounds(dev, w, cfg, rounds=args.batched_rounds)), flush=True)
        return
    max_len = P + args.tokens + 4 * (Kw + 1) + 64
    eng = GssEngine(cfg, w, max_bs=1, max_len=max_len, device=dev)
    mask_id = cfg.vocab - 1
    # logs: one row per round / AR step; the AR leg runs warmup + tokens + K + 2 steps
    dec = SelfSpecDecoder(eng, bd=bd, mask_id=mask_id, bs=1,
                          max_rounds=max(args.steps, args.tokens + Kw + 2) + args.warmup + 8)
    t0 = time.time()
    last = eng.prefill(0, emb)
    torch.cuda.synchronize()
    prefill_s = time.time() - t0
    x00 = last.float().argmax().view(1)
    log(f"prefill of {P} tokens: {prefill_s:.2f}s; first token {int(x00)}")
    # the prefill again, warm, between HIP events (it rewrites the same K/V: the prompt is the same)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    eng.prefill(0, emb)
    e1.record()
    torch.cuda.synchronize()
    pf_ms = e0.elapsed_time(e1)
    c = cfg
    gemm_flops = 2 * P * c.n_layers * c.hidden * (c.qkv_dim + c.n_heads * c.head_dim + 3 * c.ffn)
    attn_flops_pf = c.n_layers * 4 * c.n_heads * c.head_dim * P * (P + 1) // 2   # causal
    prefill = {"tokens": P, "ms": round(pf_ms, 2), "tokens_per_s": round(P / (pf_ms * 1e-3), 1),
               "gemm_flops": gemm_flops, "attn_flops": attn_flops_pf,
               "tflops_per_s": round((gemm_flops + attn_flops_pf) / (pf_ms * 1e-3) / 1e12, 1),
               "mfma_frac": round((gemm_flops + attn_flops_pf) / (pf_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
               "cold_s": round(prefill_s, 2)}
    log(f"prefill (warm): {pf_ms:.1f} ms, {prefill['tokens_per_s']} tokens/s, {prefill['tflops_per_s']} TFLOP/s")
    if args.prefill_only:
        print(json.dumps({"prefill": prefill}), flush=True)
        return

    def reset():
        eng.seq_lens[:1].fill_(P)
        dec.start(x00)

    # ---- warm up eagerly, capture the round and the AR step as HIP graphs ----------------------------------------
    reset()
    dec.round()
    reset()
    dec.ar_step()
    reset()
    dec.capture()
    torch.cuda.synchronize()
    log("graphs captured")

    # ---- AR baseline: args.tokens AR steps, graph-replayed --------------------------------------------------------
    ar_tps = ar_us = None
    ar_tokens = None
    if not args.profile_only and not args.sampled_only:
        n_ar = args.tokens + Kw + 2
        reset()
        for _ in range(args.warmup):
            dec.g_ar.replay()
        reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n_ar):
            dec.g_ar.replay()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        ar_tps, ar_us = n_ar / dt, dt / n_ar * 1e6
        ar_tokens = [int(x00)] + dec.ar_log[:n_ar, 0].cpu().tolist()
        log(f"AR: {ar_tps:.1f} tokens/s ({ar_us:.1f} us/token)")
        if args.ar_only:
            print(json.dumps({"ar_us_per_token": round(ar_us, 1), "ar_tokens_per_s": round(ar_tps, 2),
                              "steps": n_ar}), flush=True)
            return

    # ---- calibration: rounds that commit args.tokens (untimed) ---------------------------------------------------
    reset()
    rounds = 0
    committed = 1
    while committed < args.tokens:
        dec.g_round.replay()
        rounds += 1
        committed += int(dec.st.packed[0, 1]) + 2
    steps = args.steps if args.steps > 0 else rounds
    log(f"calibration: {rounds} rounds commit {committed} tokens; timing {steps} rounds")

    # ---- timed spec rounds ------------------------------------------------------------------------------------
    reset()
    for _ in range(args.warmup):
        dec.g_round.replay()
    reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        dec.g_round.replay()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    accs = dec.accept_lengths(steps)[:, 0]
    n_commit = int((accs + 2).sum())
    spec_tokens = [int(x00)] + dec.committed(steps)[0]
    tps = n_commit / dt
    round_us = dt / steps * 1e6
    log(f"spec: {n_commit} tokens in {steps} rounds, {tps:.1f} tokens/s, {round_us:.1f} us/round")
    match = None
    if ar_tokens is not None:
        n = min(len(ar_tokens), len(spec_tokens))
        match = next((i for i in range(n) if ar_tokens[i] != spec_tokens[i]), n)
        log(f"first ids: spec {spec_tokens[:8]} AR {ar_tokens[:8]}; identical prefix {match}")

    # ---- draft / verify halves (eager launches of the same kernels, graph-free timing) -------------------------
    # ---- planted acceptance ---------------------------------------------------------------------------------
    planted = None
    if ar_tokens is not None:
        g = np.random.default_rng(7)
        m_draw = np.minimum(g.geometric(0.1, size=args.tokens + 8) - 1, bd)
        ar_dev = torch.tensor(ar_tokens + [0] * (Kw + 2), dtype=torch.int32, device=dev)
        m_dev = torch.tensor(m_draw, dtype=torch.int64, device=dev)
        jj = torch.arange(1, Kw, device=dev)

        def plant():
            st = dec.st
            base = (eng.seq_lens[:1].long() - P)                      # after the x0 commit: a0's AR index
            idx = (base[:, None] + jj[None, :]).clamp(max=ar_dev.numel() - 1)
            good = ar_dev[idx]
            m = m_dev[st.ctr.clamp(max=m_dev.numel() - 1)]            # this round's planted match count
            bad = (good + 1) % cfg.vocab
            st.am[:, 1:] = torch.where(jj[None, :] <= m[:, None], good, bad)

        gp = torch.cuda.CUDAGraph()
        reset()
        dec.round(after_draft=plant)
        reset()
        with torch.cuda.graph(gp):
            dec.round(after_draft=plant)
        reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        pr = 0
        pc = 1
        while pc < args.tokens:
            gp.replay()
            pr += 1
            pc += int(dec.st.packed[0, 1]) + 2
        torch.cuda.synchronize()
        pdt = time.perf_counter() - t0
        paccs = dec.accept_lengths(pr)[:, 0]
        ptoks = [int(x00)] + dec.committed(pr)[0]
        n = min(len(ptoks), len(ar_tokens))
        planted = {"tokens_per_s": round(int((paccs + 2).sum()) / pdt, 1), "rounds": pr,
                   "mean_committed_per_round": round(float((paccs + 2).mean()), 3),
                   "speedup_vs_ar": round((int((paccs + 2).sum()) / pdt) / ar_tps, 3),
                   "ids_equal_ar_prefix": next((i for i in range(n) if ptoks[i] != ar_tokens[i]), n),
                   "note": "timing includes one host readback per round (loop control)"}
        log(f"planted: {planted}")

    # ---- sampled round (temperature 0.8, top-k 40, top-p 0.9, repetition penalty 1.1), graph-replayed -----------
    sampled = None
    if args.sampled_only or not args.profile_only:
        from gravityocr_amd.sampling import SampledSelfSpec, SamplingSpec
        torch.manual_seed(5)
        ss = SampledSelfSpec(dec, SamplingSpec(temperature=0.8, top_k=40, top_p=0.9, filter="joint",
                                                repetition_penalty=1.1))
        eng.seq_lens[:1].fill_(P)
        ss.start(x00)
        ss.round()
        gs = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gs):
            ss.round()
        eng.seq_lens[:1].fill_(P)
        ss.start(x00)
        n_s = 64
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n_s):
            gs.replay()
        torch.cuda.synchronize()
        sdt = time.perf_counter() - t0
        saccs = dec.accept_lengths(n_s)[:, 0]
        sampled = {"us_per_round": round(sdt / n_s * 1e6, 1), "rounds": n_s,
                   "tokens_per_s": round(int((saccs + 2).sum()) / sdt, 1),
                   "mean_committed_per_round": round(float((saccs + 2).mean()), 3),
                   "settings": "temperature 0.8, top-k 40, top-p 0.9 (joint), repetition penalty 1.1"}
        log(f"sampled: {sampled}")
        if args.sampled_only:
            print(json.dumps(sampled), flush=True)
            return

    # ---- draft attention roofline at the round's shape -----------------------------------------------------------
    L = P + args.tokens // 2
    d_us = attn_roofline(dev, L, Kw, eng.max_len)
    v_us = attn_roofline(dev, L, Kw, eng.max_len, n_causal=None)
    ab = attn_bytes(L, Kw)
    achieved = ab / (d_us * 1e-6) / 1e9
    tflops = attn_flops(L, Kw) / (d_us * 1e-6) / 1e12
    log(f"draft attention L={L}: {d_us:.2f} us, {achieved:.0f} GB/s, {tflops:.1f} TFLOP/s; verify {v_us:.2f} us")
    by_block = {}
    for bdb in (8, 16, 32):  # the batched config's block sizes: windows of B + 1 rows
        u, nb, fl = attn_batched_roofline(dev, W=bdb + 1)
        by_block[str(bdb)] = {"avg_us": round(u, 2), "GBs": round(nb / (u * 1e-6) / 1e9, 1),
                              "frac": round(nb / (u * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                              "mfma_tflops": round(fl / (u * 1e-6) / 1e12, 1),
                              "mfma_frac": round(fl / (u * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)}
        if bdb == 16:
            b_us, b_bytes, b_flops = u, nb, fl
    log(f"batched draft attention (32 ragged sequences): {b_us:.2f} us, {b_bytes / (b_us * 1e-6) / 1e9:.0f} GB/s; "
        f"by block size {by_block}")

    # ---- argmax / accept and KV commit at the round's shapes ---------------------------------------------------
    small = {"argmax": {}, "kv_commit": None}
    for b in (1, 8, 32):
        u, nb = argmax_roofline(dev, b)
        small["argmax"][str(b)] = {"avg_us": round(u, 2), "bytes": nb, "GBs": round(nb / (u * 1e-6) / 1e9, 1),
                                   "frac": round(nb / (u * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    u, nb = commit_roofline(dev, n_rows=Kw, L=L)
    small["kv_commit"] = {"avg_us": round(u, 2), "bytes": nb, "rows": Kw, "GBs": round(nb / (u * 1e-6) / 1e9, 1),
                          "frac": round(nb / (u * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    log(f"argmax / accept and KV commit: {small}")

    # ---- batched serving shape: 32 ragged sequences, B in {8, 16, 32} --------------------------------------------
    batched = None
    if not args.no_batched and not args.profile_only:
        batched = batched_rounds(dev, w, cfg, rounds=args.batched_rounds)

    # ---- CPU baseline: the oracle's round on the host cores, from the same 8K state -----------------------------
    cpu = None
    if not args.no_cpu and not args.profile_only:
        from oracle.decoder import DecoderConfig, KVCache, OracleDecoder
        from oracle.rounds import fulldraft_round
        torch.set_num_threads(os.cpu_count() or 1)
        ocfg = DecoderConfig(n_layers=cfg.n_layers, hidden=cfg.hidden, n_heads=cfg.n_heads, n_kv_heads=cfg.n_kv_heads,
                             head_dim=cfg.head_dim, ffn=cfg.ffn, vocab=cfg.vocab)
        wb = {k: v.bfloat16().float() for k, v in w.items()}
        om = OracleDecoder(ocfg, wb)
        reset()
        pt = eng.page_table[0, : (P + 15) // 16].long()
        cache = KVCache(cfg.n_layers)
        for l in range(cfg.n_layers):
            kk = eng.k_pages[l][pt].permute(0, 2, 1, 3).reshape(-1, cfg.n_kv_heads, cfg.head_dim)[:P]
            vv = eng.v_pages[l][pt].permute(0, 3, 1, 2).reshape(-1, cfg.n_kv_heads, cfg.head_dim)[:P]
            cache.append(l, kk.float().cpu(), vv.float().cpu())
        S, x0 = P, int(x00)
        fulldraft_round(om, cache, S, x0, bd, mask_id)      # warm-up (not counted), state restored below
        cache.truncate(P)
        n_r = n_t = 0
        t0 = time.perf_counter()
        with torch.no_grad():
            while time.perf_counter() - t0 < args.cpu_seconds or n_r < 2:
                S, x0, T, acc, _ = fulldraft_round(om, cache, S, x0, bd, mask_id)
                n_r += 1
                n_t += len(T)
        cdt = time.perf_counter() - t0
        cpu = {"value": round(n_t / cdt, 3), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"{n_r} full-draft rounds (B={bd}) of the fp32 oracle from the same {P}-token state, "
                         f"{cdt:.1f}s", "round_ms": round(cdt / n_r * 1e3, 1), **cpu_info()}
        log(f"CPU baseline: {cpu}")

    round_bytes = 2 * (1_088_618_496 + 16 * 1024 * (L + Kw) + Kw * cfg.vocab * 2)
    out = {
        "metric": "committed tokens/s bs=1 + draft/verify round µs; attn HBM GB/s vs peak",
        "value": round(tps, 2), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(round_us / 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (random-init weights, seeded N(0,1) visual embeddings and U[0,V) ids)",
        "config": {"workload": f"bs=1 self-spec full-draft rounds, 16-layer 1536-hidden GLM decoder, {P}-token "
                               f"prefix, B={bd}: {steps} timed rounds committing {n_commit} tokens",
                   "bs": 1, "prefix": P, "bd": bd, "K": Kw, "timed_rounds": steps, "timed_tokens": n_commit,
                   "parallelism": "none (one GPU)"},
        "round_us": round(round_us, 1),
        "mean_committed_per_round": round(n_commit / steps, 3),
        "accept_hist": np.bincount(accs, minlength=bd + 1).tolist(),
        "ar_tokens_per_s": None if ar_tps is None else round(ar_tps, 2),
        "ar_us_per_token": None if ar_us is None else round(ar_us, 1),
        "speedup_vs_ar": None if ar_tps is None else round(tps / ar_tps, 3),
        "spec_equals_ar_prefix": match,
        "planted": planted,
        "sampled": sampled,
        "round_hbm_frac": round(round_bytes / (round_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "prefill": prefill,
        "roofline": {"bound": "hbm", "kernel": "gss_draft_attn (block-diffusion draft attention)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": from_profile("attn_draft_bs1_8k.md", "traffic_bytes_per_call", int),
                     "mfma_util_pct_counter": from_profile("attn_draft_bs1_8k.md", "mfma_util_pct"),
                     "algorithmic_bytes": ab, "avg_us": round(d_us, 2), "L": L, "W": Kw,
                     "mfma_tflops": round(tflops, 1), "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                     "verify_avg_us": round(v_us, 2)},
        "roofline_batched": {"bound": "hbm", "kernel": "gss_draft_attn (wide kernel), 32 sequences, prefixes "
                                                       "U[1024, 12288] (seed 3), W=17, one paged pool",
                             "achieved": round(b_bytes / (b_us * 1e-6) / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(b_bytes / (b_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                             "algorithmic_bytes": b_bytes, "avg_us": round(b_us, 2),
                             "traffic": from_profile("attn_draft_batched32.md", "traffic_bytes_per_call", int),
                             "mfma_util_pct_counter": from_profile("attn_draft_batched32.md", "mfma_util_pct"),
                             "mfma_tflops": round(b_flops / (b_us * 1e-6) / 1e12, 1),
                             "mfma_frac": round(b_flops / (b_us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                             "by_block_size": by_block},
        "argmax_accept": small["argmax"],
        "kv_commit": small["kv_commit"],
        "batched": batched,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
