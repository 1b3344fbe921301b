"""Benchmark: Qwen3-8B-shape speculative verify step, tree-64, batch 64, on one MI355X.

One step = one verify step of 64 sequences, each with 2048 cached context tokens
and a 64-node depth-8 draft tree: the 36-layer target forward over the 4096 tree
rows (HIP tree attention over the paged KV cache, torch GEMMs), the LM head, the
temperature-0.8 sampler (tree rejection sampling against resident fp32 draft
probabilities; the walk computes the softmax statistics of the target rows it visits
and recomputes each probability it reads), compaction of the accepted paths' KV rows
in all 36 layers, and the read-back of the accepted lengths.  Weights are random-init
bf16 of the Qwen3-8B architecture; the cached context K/V, trees, draft distributions
and tokens are synthetic (seeded).  value = verified tokens/s = sum over the timed
steps of sum_b (accepted_len_b + 1) / elapsed.

Prints one JSON line.  `--gpus N` with N > 1 exits: the verify path runs on a single GPU.
After the verify step (outside its timed region) the line also carries the Qwen3-0.6B-shape
tree attention (`tree_attention_0p6b`) and the offline generate workload below, run in a
child process (`offline_generate`; `--no-offline-generate` skips it).

`--workload e2e` runs the offline engine benchmark instead, with the methodology
of the reference's bench.py (256 requests, prompt token ids uniform over the
vocabulary, of length U[100, 1024], max_tokens U[100, 1024], temperature 0.6,
ignore_eos, one warmup
generate, wall-clock timing): Qwen3-0.6B architecture with random-init weights,
drafting with a random-init EAGLE-3 head (T = 32 tree nodes) or without
speculation (`--spec none`); value = output tokens/s.

`--workload kernels` times each kernel of the path at its own workload (chain
sampler, n-gram drafter, tree attention at the Qwen3-0.6B shape, and the KV
scatter, compaction, softmax, tree rejection walk and draft top-k at the verify-step
shape) against the oracle on the host, one JSON line per workload.

`--workload power` runs loads back to back for a few seconds each while sampling the
socket power (`amd-smi metric -p`) and shader clock (`rocm-smi --showclocks`): idle,
tree attention at the verify-step layer shape and in causal prefill, a bf16 GEMM and a
device copy.  From the GEMM (energy per MFMA FLOP) and the copy (energy per HBM byte)
it derives the shortest time the power cap allows for the verify-step attention layer.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nano-vllm-x_amd"))
sys.path.insert(0, ROOT)

METRIC = "verified tokens/s, Qwen3-8B-shape tree-64 verify b=64; sampler HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
PMC_SUMMARY = os.path.join(ROOT, "profiles", "tree_attention_verify8b_pmc.txt")
ATTN_SOURCE = os.path.join(ROOT, "nano-vllm-x_amd", "csrc", "attention.hip")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--tree-nodes", type=int, default=64)
    ap.add_argument("--tree-depth", type=int, default=8)
    ap.add_argument("--context", type=int, default=2048)
    ap.add_argument("--temperature", type=float, default=0.8)
    ap.add_argument("--model", default="Qwen3-8B")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seqs", type=int, default=6,
                    help="sequences in the CPU-baseline sample (0 disables it)")
    ap.add_argument("--parity-seqs", type=int, default=8,
                    help="sequences of the integrated step checked against the oracle (0: off)")
    ap.add_argument("--small-tree-attention", action=argparse.BooleanOptionalAction, default=True,
                    help="also time tree attention at the Qwen3-0.6B shape (batch 32, 32-node "
                         "trees, ctx 1024-4096) with a parity check on 2 sequences")
    ap.add_argument("--offline-generate", action=argparse.BooleanOptionalAction, default=True,
                    help="after the verify step, run the offline generate workload (--workload e2e) "
                         "in a child process and add its summary to the JSON line")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a 1 GiB device copy (HBM counter calibration)")
    ap.add_argument("--workload", choices=("verify", "e2e", "kernels", "power"), default="verify")
    ap.add_argument("--power-secs", type=float, default=4.0,
                    help="seconds of back-to-back launches per load in --workload power")
    ap.add_argument("--spec", choices=("eagle3", "ngram", "none"), default="eagle3",
                    help="e2e: speculative method")
    ap.add_argument("--e2e-seqs", type=int, default=256)
    ap.add_argument("--e2e-max-in", type=int, default=1024)
    ap.add_argument("--e2e-max-out", type=int, default=1024)
    ap.add_argument("--eagle-topk", type=int, default=8)
    ap.add_argument("--eagle-depth", type=int, default=6)
    ap.add_argument("--graphs", action=argparse.BooleanOptionalAction, default=True,
                    help="e2e: replay the steps from captured HIP graphs (the reference bench "
                         "runs with enforce_eager=False); --no-graphs runs them eagerly")
    return ap.parse_args()


def run_e2e(args):
    """Offline output throughput through LLM.generate (reference bench.py:9-28)."""
    from random import randint, seed
    import torch
    from nanovllm import LLM, SamplingParams
    from nanovllm.models.qwen3 import qwen3_config

    seed(0)
    cfg = qwen3_config("Qwen3-0.6B")
    cfg.eos_token_id = -1
    T = 32 if args.tree_nodes == 64 else args.tree_nodes  # config 5 default: 32-node trees
    kw = {}
    if args.spec == "eagle3":
        kw = dict(speculative_method="eagle3", num_speculative_tokens=T - 1,
                  eagle_topk=args.eagle_topk, eagle_depth=args.eagle_depth)
    elif args.spec == "ngram":
        kw = dict(speculative_method="ngram", num_speculative_tokens=5)
    blocks = args.e2e_seqs * ((args.e2e_max_in + args.e2e_max_out + 64) // 256 + 2) + 64
    llm = LLM("unused", hf_config=cfg, max_model_len=4096, num_kvcache_blocks=blocks,
              seed=args.seed, enforce_eager=not args.graphs, **kw)
    # prompt ids uniform over the whole vocabulary (the reference's bench.py:17 draws
    # them from [0, 10000])
    prompt_token_ids = [[randint(0, cfg.vocab_size - 1) for _ in range(randint(100, args.e2e_max_in))]
                        for _ in range(args.e2e_seqs)]
    sampling_params = [SamplingParams(temperature=0.6, ignore_eos=True,
                                      max_tokens=randint(100, args.e2e_max_out))
                       for _ in range(args.e2e_seqs)]
    llm.generate([[1, 2, 3, 4]], SamplingParams(max_tokens=8), use_tqdm=False)
    stats = llm.model_runner.spec_stats
    stats.update(verify_rows=0, accepted=0, accepted_hist={})
    torch.cuda.synchronize()
    t = time.perf_counter()
    # the progress bar (stderr) only redraws; the reference runs without it
    llm.generate(prompt_token_ids, sampling_params, use_tqdm=True)
    torch.cuda.synchronize()
    t = time.perf_counter() - t
    total = sum(sp.max_tokens for sp in sampling_params)
    out = {
        "metric": "output tokens/s, offline generate (reference bench.py workload)",
        "value": total / t, "unit": "tokens/s", "n_gpus": 1, "higher_is_better": True,
        "elapsed_s": t, "output_tokens": total, "dtype": "bf16",
        "data": "synthetic (random-init weights, prompt token ids uniform over the vocabulary)",
        "config": {"workload": "offline generate", "model": "Qwen3-0.6B-shape", "requests": args.e2e_seqs,
                   "input_len": f"U[100,{args.e2e_max_in}]", "output_len": f"U[100,{args.e2e_max_out}]",
                   "temperature": 0.6, "speculative": args.spec, "hip_graphs": args.graphs,
                   **({"tree_nodes": T, "eagle_topk": args.eagle_topk, "eagle_depth": args.eagle_depth,
                       "draft_vocab": llm.model_runner.draft.lm_head.weight.shape[0]}
                      if args.spec == "eagle3" else {})},
        "mean_accepted_per_verify": stats["accepted"] / max(stats["verify_rows"], 1),
        "verify_rows": stats["verify_rows"],
    }
    print(json.dumps(out), flush=True)


def kernel_source_digest():
    """sha256 of the attention kernel's source: the committed counter profile names
    the source it was measured on."""
    import hashlib
    with open(ATTN_SOURCE, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def read_pmc_traffic():
    """HBM bytes per attention launch from the committed rocprofv3 --pmc summary, or
    (None, reason) when the summary is missing or was measured on another source of
    the attention kernel."""
    fields = {}
    try:
        with open(PMC_SUMMARY) as f:
            for line in f:
                if ":" in line and not line.startswith((" ", "#")):
                    k, v = line.split(":", 1)
                    fields[k.strip()] = v.strip()
    except OSError:
        return None, "no counter profile"
    if fields.get("kernel_source_sha256") != kernel_source_digest():
        return None, "counter profile measured on another attention.hip (stale); traffic not reported"
    try:
        return float(fields["traffic_bytes_per_launch"]), None
    except (KeyError, ValueError):
        return None, "counter profile without traffic_bytes_per_launch"


def build_step(args, torch, dev):
    import numpy as np
    from nanovllm import _C
    from nanovllm.layers.sampler import RejectionSampler
    from nanovllm.models.qwen3 import Qwen3ForCausalLM, qwen3_config, random_init_
    from nanovllm.spec.kv_compact import kv_compact
    from nanovllm.spec.tree import random_tree
    from nanovllm.utils.context import set_context, reset_context
    from nanovllm.utils.synthetic import VerifyBatch

    _C.lib()
    cfg = qwen3_config(args.model)
    torch.set_default_dtype(torch.bfloat16)
    with torch.device(dev):
        model = Qwen3ForCausalLM(cfg)
    torch.set_default_dtype(torch.float32)
    random_init_(model, seed=args.seed)
    model.eval()

    B, T = args.batch, args.tree_nodes
    rng = np.random.default_rng(args.seed)
    trees = [random_tree(T, args.tree_depth, rng) for _ in range(B)]
    vb = VerifyBatch([args.context] * B, trees, 256, rng)
    L, Hkv, D = cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim
    kv_cache = torch.empty(2, L, vb.num_blocks, 256, Hkv, D, dtype=torch.bfloat16, device=dev)
    gen = torch.Generator(device=dev).manual_seed(args.seed + 1)
    for i in range(2):
        for l in range(L):
            kv_cache[i, l].normal_(0.0, 1.0, generator=gen)
    for l, attn in enumerate(model.attention_layers()):
        attn.k_cache, attn.v_cache = kv_cache[0, l], kv_cache[1, l]

    V = cfg.vocab_size
    # Resident draft distributions (one row per node) and tree tokens drawn from them.
    Q = torch.empty(B, T, V, dtype=torch.float32, device=dev)
    for b in range(B):
        Q[b].normal_(0.0, 2.0, generator=gen)
        Q[b] = torch.softmax(Q[b] / args.temperature, -1)
    parents = torch.from_numpy(np.stack(trees)).to(dev)
    tokens = torch.empty(B, T, dtype=torch.int64, device=dev)
    tokens[:, 0] = torch.randint(0, V, (B,), generator=gen, device=dev)
    child = torch.arange(1, T, device=dev)
    for b in range(B):
        # node i's token is an independent draw from its parent's draft row
        drawn = torch.multinomial(Q[b], T, replacement=True, generator=gen)  # [T rows, T draws]
        tokens[b, 1:] = drawn[parents[b, 1:].long(), child]
    tokens32 = tokens.to(torch.int32)

    t = lambda a, dt=torch.int32: torch.from_numpy(a).to(device=dev, dtype=dt)
    input_ids = tokens.view(-1)
    positions = t(vb.positions, torch.int64)
    slot_mapping, cu_q = t(vb.slot_mapping), t(vb.cu_q)
    context_lens, block_tables = t(vb.context_lens), t(vb.bt)
    tree_mask = t(vb.masks, torch.int64)
    ctx = t(vb.ctx)
    temps = torch.full((B,), args.temperature, dtype=torch.float32, device=dev)
    sampler = RejectionSampler()
    ugen = torch.Generator(device=dev).manual_seed(args.seed + 2)

    @torch.inference_mode()
    def forward():
        """The target forward over the tree rows and the LM head: logits [B*T, V]."""
        set_context(False, cu_seqlens_q=cu_q, slot_mapping=slot_mapping, context_lens=context_lens,
                    block_tables=block_tables, tree_mask=tree_mask, max_seqlen_q=T,
                    max_context_len=int(vb.context_lens.max()))
        hidden = model(input_ids, positions)
        logits = model.compute_logits(hidden)
        reset_context()
        return logits

    @torch.inference_mode()
    def step(capture=None):
        """One verify step; returns [B, 1 + T] int32 on the host: accepted_len, then
        the path.  capture (a dict, outside the timed region) receives the step's
        logits, uniforms and sampler outputs, and a copy of the KV cache from before
        the compaction, for the parity check.  Raises if the walk failed for any
        sequence (accepted_len -1)."""
        logits = forward()
        U = torch.rand(B, T, device=dev, generator=ugen)
        Uf = torch.rand(B, device=dev, generator=ugen)
        stats = capture["stats"] if capture is not None else None
        path, acc, out_tok, nxt = sampler(logits, temps, Q, tokens32, parents, U, Uf,
                                          stats_out=stats)
        if capture is not None:
            lay, pages = capture["kv_layers"], capture["kv_pages"]
            capture.update(logits=logits, U=U, Uf=Uf, path=path, acc=acc, out_tokens=out_tok,
                           next_token=nxt, kv_before=kv_cache[:, lay][:, :, pages].clone())
        kv_compact(kv_cache[0], kv_cache[1], block_tables, ctx, path, acc)
        res = torch.cat([acc[:, None], path], dim=1).cpu()
        if bool((res[:, 0] < 0).any()):
            raise RuntimeError("tree rejection walk failed (accepted_len -1) for batch rows "
                               f"{torch.nonzero(res[:, 0] < 0).flatten().tolist()}")
        return res

    state = dict(model=model, kv_cache=kv_cache, vb=vb, Q=Q, tokens=tokens32, tokens64=tokens,
                 parents=parents, cfg=cfg, temps=temps, forward=forward)
    return step, state


def host_threads():
    """Threads for the host-side oracle: every CPU this process may run on, capped by
    OMP_NUM_THREADS when it is set (the host's CPU share for the job)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(omp))) if omp.isdigit() and int(omp) > 0 else n


def host_info(torch):
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    aff = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None
    return {"nproc": os.cpu_count(), "affinity_cpus": aff,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "cpu_model": model,
            "torch_version": torch.__version__}


def cpu_baseline(args, torch, state, nseq):
    """The same verify step restated on the host for a sample of `nseq` sequences:
    torch-CPU fp32 dense layers plus the oracle's paged tree attention, softmax,
    rejection sampler and compaction.  Returns (verified tokens/s, cores, seconds)."""
    import numpy as np
    from oracle import attention as oatt, kvcache as okv, sampler as osamp

    cores = host_threads()
    torch.set_num_threads(cores)
    model, vb, cfg = state["model"], state["vb"], state["cfg"]
    L, Hq, Hkv, D = cfg.num_hidden_layers, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    bs = 256
    sel = list(range(nseq))
    rows = np.concatenate([np.arange(vb.cu_q[b], vb.cu_q[b + 1]) for b in sel])
    # local copy of the selected sequences' pages (all layers), renumbered 0..n-1
    used = sorted({int(x) for b in sel for x in vb.bt[b] if x >= 0})
    remap = {old: i for i, old in enumerate(used)}
    bt = np.array([[remap.get(int(x), -1) for x in vb.bt[b]] for b in sel], np.int32)
    idx = torch.tensor(used, device=state["kv_cache"].device)
    kc = state["kv_cache"][0][:, idx].float().cpu().numpy()  # [L, n, bs, Hkv, D]
    vc = state["kv_cache"][1][:, idx].float().cpu().numpy()
    W = {n: p.detach().float().cpu() for n, p in model.named_parameters()}
    ids = state["tokens"].view(-1).cpu()[rows].long()
    pos = torch.from_numpy(vb.positions[rows]).long()
    slots = np.concatenate([okv.slot_of(bt[i], vb.ctx[b] + np.arange(vb.qlens[b]), bs)
                            for i, b in enumerate(sel)])
    cu = np.zeros(nseq + 1, np.int32)
    cu[1:] = np.cumsum(vb.qlens[sel])
    ctxl = vb.context_lens[sel]
    masks = np.concatenate([vb.masks[vb.cu_q[b]:vb.cu_q[b + 1]] for b in sel]).view(np.uint64)
    Qs = state["Q"][:nseq].cpu().numpy()
    par = state["parents"][:nseq].cpu().numpy()
    toks = state["tokens"][:nseq].cpu().numpy()
    rng = np.random.default_rng(7)
    U = rng.random((nseq, vb.T)).astype(np.float32)
    Uf = rng.random(nseq).astype(np.float32)
    theta = 1000000.0
    inv_freq = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float) / D))
    freqs = torch.outer(pos.float(), inv_freq)
    cos, sin = freqs.cos().unsqueeze(1), freqs.sin().unsqueeze(1)

    def rms(x, w, eps=cfg.rms_norm_eps):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w

    def rope(x):
        x1, x2 = x.chunk(2, -1)
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), -1)

    t0 = time.perf_counter()
    with torch.inference_mode():
        h = W["model.embed_tokens.weight"][ids]
        res = None
        for l in range(L):
            pre = f"model.layers.{l}."
            if res is None:
                res = h
            else:
                res = h + res
            x = rms(res, W[pre + "input_layernorm.weight"])
            qkv = x @ W[pre + "self_attn.qkv_proj.weight"].T
            q, k, v = qkv.split([Hq * D, Hkv * D, Hkv * D], -1)
            q = rope(rms(q.view(-1, Hq, D), W[pre + "self_attn.q_norm.weight"]))
            k = rope(rms(k.view(-1, Hkv, D), W[pre + "self_attn.k_norm.weight"]))
            kl, vl = kc[l], vc[l]
            okv.store_kvcache(k.numpy(), v.view(-1, Hkv, D).numpy(), kl, vl, slots)
            o = oatt.paged_attention(q.numpy(), kl, vl, bt, cu, ctxl, masks, D ** -0.5, bs)
            h = torch.from_numpy(o).view(-1, Hq * D) @ W[pre + "self_attn.o_proj.weight"].T
            res = h + res
            x = rms(res, W[pre + "post_attention_layernorm.weight"])
            gate, up = (x @ W[pre + "mlp.gate_up_proj.weight"].T).chunk(2, -1)
            h = (torch.nn.functional.silu(gate) * up) @ W[pre + "mlp.down_proj.weight"].T
        x = rms(h + res, W["model.norm.weight"])
        logits = (x @ W["lm_head.weight"].T).numpy()
        P = osamp.temperature_softmax(logits, np.full(len(rows), args.temperature, np.float32))
        path, acc, _, _ = osamp.rejection_sample_tree(P.reshape(nseq, vb.T, -1), Qs, toks, par, U,
                                                      Uf, np.zeros(nseq, bool))
        okv.kv_compact(kc, vc, bt, vb.ctx[sel], path, acc, bs)
    dt = time.perf_counter() - t0
    return float((acc + 1).sum()) / dt, cores, dt


def plant_greedy_spines(torch, state, nplant, depth):
    """Make the first nplant sequences greedy (temperature 0) and plant, along the
    root-to-leaf path to each tree's first deepest node, the target's own greedy
    chain: the token of the path's node d is the argmax of the target row of node
    d - 1.  A row depends on the tokens of its ancestors, so the chain is built depth
    by depth, one target forward per depth.  Then the greedy walk accepts the whole
    path (accepted_len = depth, unless an earlier sibling carries the same token or
    the argmax is tied) and compaction moves depth rows in every layer.  Returns the
    planted paths and a function that restores the tokens and temperatures."""
    import numpy as np
    from nanovllm.spec.tree import depths as tree_depths

    tok64, tok32, temps = state["tokens64"], state["tokens"], state["temps"]
    saved = (tok64.clone(), temps.clone())
    T = tok64.shape[1]
    parents = state["parents"].cpu().numpy()
    paths = []
    for b in range(nplant):
        d = tree_depths(parents[b])
        node = int(np.argmax(d))
        path = [node]
        while path[-1] != 0:
            path.append(int(parents[b][path[-1]]))
        paths.append(path[::-1])
    temps[:nplant] = 0.0
    with torch.inference_mode():
        for lvl in range(1, 1 + min([depth] + [len(p) - 1 for p in paths]) if paths else 1):
            logits = state["forward"]()
            rows = torch.tensor([b * T + p[lvl - 1] for b, p in enumerate(paths)],
                                device=logits.device)
            am = logits[rows].float().argmax(-1)
            for b, p in enumerate(paths):
                tok64[b, p[lvl]] = am[b]
            tok32.copy_(tok64.to(torch.int32))
    torch.cuda.synchronize()

    def restore():
        tok64.copy_(saved[0])
        tok32.copy_(saved[0].to(torch.int32))
        temps.copy_(saved[1])

    return paths, restore


def integrated_parity(args, torch, state, step, nseq):
    """One more verify step (outside the timed region), checked against the oracle on
    the step's own data for its first nseq sequences.  The first half of them are
    made greedy with the target's own greedy chain planted on a root-to-leaf path
    (plant_greedy_spines), so the walk accepts deep paths and compaction moves that
    many rows in all layers; the rest stay stochastic at the bench temperature.  The
    walk computes the statistics of the rows it visits and reports them; the oracle
    walks the probabilities of the GPU's logits (nvx_softmax_from_stats with those
    statistics on the visited rows and the statistics pass's elsewhere, all checked
    against the float64 softmax; the fp32 logits for greedy rows) with the same draft
    rows, tokens, tree and uniforms, and compacts a copy of the pre-compaction KV pages
    of the first and last layer along the GPU's paths.  Integer outputs and KV bytes
    must be equal, and the visited rows must be exactly the sampled sequences' accepted
    paths.  Returns the parity record."""
    import numpy as np
    from nanovllm.layers.sampler import softmax_from_stats, softmax_stats
    from oracle import kvcache as okv, sampler as osamp

    vb, cfg, kv = state["vb"], state["cfg"], state["kv_cache"]
    B, T, V, L = args.batch, args.tree_nodes, cfg.vocab_size, cfg.num_hidden_layers
    dev = kv.device
    nplant = nseq // 2
    paths, restore = plant_greedy_spines(torch, state, nplant, args.tree_depth)
    try:
        used = sorted({int(x) for b in range(nseq) for x in vb.bt[b] if x >= 0})
        remap = {old: i for i, old in enumerate(used)}
        bt_local = np.array([[remap.get(int(x), -1) for x in vb.bt[b]] for b in range(nseq)],
                            np.int32)
        layers = [0, L - 1]
        cap = {"kv_layers": torch.tensor(layers, device=dev),
               "kv_pages": torch.tensor(used, device=dev),
               "stats": torch.full((B * T, 2), float("nan"), device=dev)}
        step(capture=cap)
        torch.cuda.synchronize()
        rows = cap["logits"][:nseq * T]
        seq_temps = state["temps"][:nseq].clone()
        rtemps = seq_temps.repeat_interleave(T)
        stats = softmax_stats(rows, rtemps)
        lazy = cap["stats"][:nseq * T]
        visited = ~torch.isnan(lazy[:, 0])
        stats[visited] = lazy[visited]
        P = softmax_from_stats(rows, rtemps, stats).cpu().numpy()
        Pref = osamp.temperature_softmax(rows.float().cpu().numpy(), rtemps.cpu().numpy())
        softmax_ok = bool(np.allclose(P, Pref, rtol=1e-5, atol=1e-35))
        greedy = seq_temps.cpu().numpy() == 0
        gpu = {k: cap[k][:nseq].cpu().numpy() for k in ("path", "acc", "out_tokens", "next_token")}
        ref_path, ref_acc, ref_tok, ref_next = osamp.rejection_sample_tree(
            P.reshape(nseq, T, V), state["Q"][:nseq].cpu().numpy(),
            state["tokens"][:nseq].cpu().numpy(), state["parents"][:nseq].cpu().numpy(),
            cap["U"][:nseq].cpu().numpy(), cap["Uf"][:nseq].cpu().numpy(), greedy)
        # KV compaction of the sampled sequences' pages, layers 0 and L-1
        as_u16 = lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16)  # noqa: E731
        before = as_u16(cap["kv_before"])                    # [2, 2 layers, pages, bs, Hkv, D]
        after = as_u16(kv[:, cap["kv_layers"]][:, :, cap["kv_pages"]])
        k_ref, v_ref = before[0].copy(), before[1].copy()
        okv.kv_compact(k_ref, v_ref, bt_local, vb.ctx[:nseq], gpu["path"], gpu["acc"], 256)
        kv_ok = bool(np.array_equal(after[0], k_ref) and np.array_equal(after[1], v_ref))
        moved = int(np.clip(gpu["acc"], 0, None).sum())
        want_vis = np.zeros(nseq * T, bool)
        for b in range(nseq):
            if seq_temps[b].item() > 0:
                want_vis[b * T + gpu["path"][b, :gpu["acc"][b] + 1]] = True
        visited_ok = bool(np.array_equal(visited.cpu().numpy(), want_vis))
    finally:
        restore()
    return {"path": bool(np.array_equal(gpu["path"], ref_path)),
            "accepted_len": bool(np.array_equal(gpu["acc"], ref_acc)),
            "tokens": bool(np.array_equal(gpu["out_tokens"], ref_tok)),
            "next_token": bool(np.array_equal(gpu["next_token"], ref_next)),
            "kv_compact": kv_ok, "softmax_within_1e-5": softmax_ok,
            "lazy_stats_rows_are_paths": visited_ok,
            "accepted": [int(a) for a in gpu["acc"]],
            "greedy": [bool(g) for g in greedy],
            "planted_path_len": [len(p) - 1 for p in paths],
            "kv_rows_moved_per_layer": moved,
            "sample": f"first {nseq} of {B} sequences of one more verify step, the first "
                      f"{nplant} greedy with the target's greedy chain planted on a "
                      f"root-to-leaf path ({max([0] + [len(p) - 1 for p in paths])} extra target "
                      f"forwards before it, untimed), the rest stochastic at T = {args.temperature}; KV "
                      f"of layers {layers[0]} and {layers[1]}"}


def walk_rows(parents, path_acc):
    """Rows the tree walk must read in one step (stochastic mode): every rejected child
    costs one residual pass over its node's target and draft rows; the final draw
    reuses the residual of the last rejection, so it reads a row only when the walk
    ends at a leaf (its target row).  Returns (target rows, draft rows).  The walk
    tests children in ascending order, so at a node on the path every child before the
    accepted one was rejected, and at the last node every child was."""
    import numpy as np
    B, T = parents.shape
    kids = [[np.nonzero(parents[b] == n)[0] for n in range(T)] for b in range(B)]
    p_rows = q_rows = 0
    for b in range(B):
        acc = int(path_acc[b, 0])
        path = path_acc[b, 1:2 + acc]
        for d in range(acc + 1):
            ch = kids[b][int(path[d])]
            rej = int((ch < path[d + 1]).sum()) if d < acc else len(ch)
            p_rows += rej + (1 if d == acc and rej == 0 else 0)
            q_rows += rej
    return p_rows, q_rows


def gpu_launch_us(torch, fn, timer, iters=20, warm=3):
    """Average µs per launch of the library kernel `timer` over `iters` calls of fn
    (after `warm` untimed calls), from the library's HIP events on the launch stream."""
    from nanovllm import _C
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    _C.timing_reset()
    _C.timing_enable(True)
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    _C.timing_enable(False)
    ms, n = _C.timing_read(timer)
    return ms / n * 1e3


def attention_small_tree(torch, dev, seed, gpu_us, check_seqs):
    """Tree attention at the Qwen3-0.6B shape (16/8 heads, d 128): 32 sequences with
    1024-4096 cached tokens and 32-node depth-6 trees in randomly scattered 256-token
    pages.  Times the launch (split-KV main kernel and merge) with the library's
    HIP-event timer and checks the first check_seqs sequences against the oracle
    (2e-2 absolute).  Returns a record."""
    import numpy as np
    from nanovllm import _C
    from nanovllm.layers.attention import tree_attention
    from nanovllm.utils.synthetic import VerifyBatch
    from oracle import attention as oatt

    B, T, Hq, Hkv, D = 32, 32, 16, 8, 128
    rng = np.random.default_rng(seed + 2)
    vb = VerifyBatch.random(B, (1024, 4096), T, 6, 256, rng)
    g = torch.Generator().manual_seed(seed + 2)
    kc = (torch.randn(vb.num_blocks, 256, Hkv, D, generator=g)).to(torch.bfloat16)
    vc = (torch.randn(vb.num_blocks, 256, Hkv, D, generator=g)).to(torch.bfloat16)
    N = int(vb.cu_q[-1])
    q = torch.randn(N, Hq, D, generator=g).to(torch.bfloat16)
    t = lambda a, dt=torch.int32: torch.from_numpy(a).to(dev, dt)  # noqa: E731
    qd, kcd, vcd = q.to(dev), kc.to(dev), vc.to(dev)
    a_args = (qd, kcd, vcd, t(vb.bt), t(vb.cu_q), t(vb.context_lens), D ** -0.5,
              t(vb.masks, torch.int64), T, int(vb.context_lens.max()))
    us = gpu_us(lambda: tree_attention(*a_args), _C.TIMER_TREE_ATTENTION)
    o = tree_attention(*a_args).float().cpu().numpy()
    ns = check_seqs
    rows = int(vb.cu_q[ns])
    t0 = time.perf_counter()
    ref = oatt.paged_attention(
        q[:rows].float().numpy(), kc.float().numpy(), vc.float().numpy(), vb.bt[:ns],
        vb.cu_q[:ns + 1], vb.context_lens[:ns], vb.masks[:rows].view(np.uint64), D ** -0.5, 256)
    cus = (time.perf_counter() - t0) * 1e6
    err = float(np.abs(o[:rows] - ref).max())
    nbytes = float(vb.context_lens.sum()) * Hkv * D * 2 * 2 + 2.0 * N * Hq * D * 2
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"config": "Qwen3-0.6B shape (16/8 heads, d 128), batch 32, ctx 1024-4096, "
                      "32-node depth-6 trees",
            "gpu_us": us, "algorithmic_bytes": nbytes, "GBs": gbs, "frac": gbs / HBM_PEAK_GBS,
            "cpu_oracle_us": cus * B / ns, "sample": f"{ns} of {B} sequences, scaled",
            "parity_with_oracle": err <= 2e-2, "max_abs_err": err,
            "note": f"max abs error vs oracle on the sample {err:.2e} (tolerance 2e-2)"}


def run_kernels(args):
    """Each kernel of the path at its own workload: the chain sampler (batch 8, k = 4),
    the n-gram drafter (64 histories of 1024-4096 tokens, plus a scaled run), tree
    attention at the Qwen3-0.6B shape (batch 32, 32-node trees) and in causal prefill
    (Qwen3-8B heads, 4 prompts of 2048 tokens), and the KV scatter,
    compaction (worst case), softmax, tree rejection walk and draft top-k at the
    Qwen3-8B verify-step shape.  GPU time per launch comes from the library's HIP-event
    timers; the oracle runs on the host over the same inputs (or a stated sample, scaled
    to the whole input) and checks the GPU result.  Prints one JSON line per workload."""
    import numpy as np
    import torch
    from nanovllm import _C
    from nanovllm.layers.attention import store_kvcache, tree_attention
    from nanovllm.layers.sampler import (rejection_sample_chain, rejection_sample_tree,
                                         rejection_sample_tree_logits,
                                         rejection_sample_tree_logits_lazy, softmax_from_stats,
                                         softmax_stats, temperature_softmax, topk_logprobs)
    from nanovllm.spec.kv_compact import kv_compact
    from nanovllm.spec.ngram import ngram_propose
    from nanovllm.spec.tree import chain_parents, random_tree
    from nanovllm.utils.synthetic import VerifyBatch, ngram_histories, pack_histories
    from oracle import attention as oatt, draft as odraft, kvcache as okv, ngram as ong
    from oracle import sampler as osamp

    _C.lib()
    dev = torch.device("cuda:0")
    cores = host_threads()
    torch.set_num_threads(cores)
    V = 151936

    def gpu_us(fn, timer, iters=20, warm=3):
        return gpu_launch_us(torch, fn, timer, iters, warm)

    def cpu_us(fn, reps=1):
        t0 = time.perf_counter()
        for _ in range(reps):
            out = fn()
        return (time.perf_counter() - t0) / reps * 1e6, out

    def emit(kernel, workload, us, nbytes, cpu, sample, parity, note=None):
        rec = {"workload": "kernels", "kernel": kernel, "config": workload, "gpu_us": us,
               "algorithmic_bytes": nbytes,
               "GBs": nbytes / (us * 1e-6) / 1e9 if nbytes else None,
               "frac_of_hbm_peak": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS if nbytes else None,
               "cpu_oracle_us": cpu, "cpu_cores": cores, "cpu_sample": sample,
               "parity_with_oracle": parity}
        if note:
            rec["note"] = note
        print(json.dumps(rec), flush=True)

    def log(msg):
        print(f"[bench kernels] {msg}", file=sys.stderr, flush=True)

    # -- chain rejection sampling, batch 8, k = 4 (stochastic and greedy)
    log("chain sampler")
    g = torch.Generator().manual_seed(args.seed)
    B, k = 8, 4
    P = torch.softmax(torch.randn(B, k + 1, V, generator=g) * 2.0, -1)
    Q = torch.softmax(torch.randn(B, k, V, generator=g) * 2.0, -1)
    drafts = torch.stack([torch.multinomial(Q[b], 1, generator=g)[:, 0] for b in range(B)]).int()
    rng = np.random.default_rng(args.seed)
    U = torch.from_numpy(rng.random((B, k)).astype(np.float32))
    Uf = torch.from_numpy(rng.random(B).astype(np.float32))
    Pd, Qd, Dd, Ud, Ufd = (t.to(dev) for t in (P, Q, drafts, U, Uf))
    for greedy in (False, True):
        gmask = torch.full((B,), greedy, dtype=torch.bool)
        gd = gmask.to(dev)
        us = gpu_us(lambda: rejection_sample_chain(Pd, Qd, Dd, Ud, Ufd, gd), _C.TIMER_REJECTION)
        acc, rec, bon, toks = (t.cpu().numpy() for t in rejection_sample_chain(Pd, Qd, Dd, Ud, Ufd, gd))
        cus, ref = cpu_us(lambda: osamp.rejection_sample_chain(P.numpy(), Q.numpy(), drafts.numpy(),
                                                               U.numpy(), Uf.numpy(), gmask.numpy()))
        ok = all(np.array_equal(a, np.asarray(r)) for a, r in zip((acc, rec, bon, toks), ref))
        emit("rejection_sample_chain", f"batch 8, k = 4, vocab {V}, fp32, "
             f"{'greedy' if greedy else 'stochastic'}", us, None, cus, "the whole input", ok,
             f"latency-bound walk: reads only the rows it visits, at most all P and Q rows "
             f"({B * (2 * k + 1) * V * 4 / 1e6:.1f} MB)")

    # -- n-gram drafter: 64 histories of 1024-4096 tokens, and a scaled run
    for name, nseq, lo, hi, sample in (("batch 64, lengths 1024-4096", 64, 1024, 4096, 64),
                                       ("scaled: batch 256, lengths 16384-65536", 256, 16384, 65536, 16)):
        log(f"n-gram drafter ({name})")
        hist = ngram_histories(nseq, lo, hi, V, np.random.default_rng(args.seed + 1))
        flat, offs = pack_histories(hist)
        td, od = torch.from_numpy(flat).to(dev), torch.from_numpy(offs).to(dev)
        us = gpu_us(lambda: ngram_propose(td, od, 3, 1, 5), _C.TIMER_NGRAM)
        draft, dlen = (t.cpu().numpy() for t in ngram_propose(td, od, 3, 1, 5))
        sflat, soffs = pack_histories(hist[:sample])
        cus, (rdraft, rlen) = cpu_us(lambda: ong.ngram_propose(sflat, soffs, 3, 1, 5))
        ok = np.array_equal(draft[:sample], rdraft) and np.array_equal(dlen[:sample], rlen)
        emit("ngram_propose", f"{name}, k = 5, n = 3..1", us, float(4 * len(flat) + 8 * nseq * 5),
             cus * nseq / sample, f"{sample} of {nseq} histories, scaled to {nseq}", ok)

    # -- tree attention, Qwen3-0.6B shape: batch 32, ctx 1024-4096, 32-node depth-6 trees
    log("tree attention (0.6B shape)")
    c3 = attention_small_tree(torch, dev, args.seed, gpu_us, check_seqs=4)
    emit("tree_attention", c3["config"], c3["gpu_us"], c3["algorithmic_bytes"],
         c3["cpu_oracle_us"], c3["sample"], c3["parity_with_oracle"], c3["note"])

    # -- causal paged prefill (the attention kernel with no tree mask), Qwen3-8B heads:
    #    4 prompts of 2048 tokens whose K/V are already in the cache
    log("tree attention (causal prefill, 8B heads)")
    t = lambda a, dt=torch.int32: torch.from_numpy(a).to(dev, dt)  # noqa: E731
    B, Tq, Hq, Hkv, D = 4, 2048, 32, 8, 128
    rng = np.random.default_rng(args.seed + 5)
    vb = VerifyBatch([0] * B, [chain_parents(Tq)] * B, 256, rng)
    g = torch.Generator().manual_seed(args.seed + 5)
    kc = torch.randn(vb.num_blocks, 256, Hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(vb.num_blocks, 256, Hkv, D, generator=g).to(torch.bfloat16)
    q = torch.randn(B * Tq, Hq, D, generator=g).to(torch.bfloat16)
    p_args = (q.to(dev), kc.to(dev), vc.to(dev), t(vb.bt), t(vb.cu_q), t(vb.context_lens),
              D ** -0.5, None, Tq, Tq)
    us = gpu_us(lambda: tree_attention(*p_args), _C.TIMER_TREE_ATTENTION)
    o = tree_attention(*p_args).float().cpu().numpy()
    s0, nr = Tq - 64, 64  # sample: the last 64 query rows of sequence 0 (keys <= s0 + i)
    cus, ref = cpu_us(lambda: oatt.paged_attention(
        q[s0:s0 + nr].float().numpy(), kc.float().numpy(), vc.float().numpy(), vb.bt[:1],
        np.array([0, nr], np.int32), np.array([s0 + nr], np.int32), None, D ** -0.5, 256))
    err = float(np.abs(o[s0:s0 + nr] - ref).max())
    pairs = B * Tq * (Tq + 1) / 2  # (query, visible key) pairs
    flops = 4.0 * Hq * D * pairs
    tflops = flops / (us * 1e-6) / 1e12
    emit("tree_attention (causal prefill)", "Qwen3-8B heads (32/8, d 128), 4 prompts of 2048 "
         "tokens, causal", us, None, cus * pairs / (nr * (s0 + (nr + 1) / 2)),
         f"{nr} of {B * Tq} query rows (the last of sequence 0), scaled by visible keys",
         err <= 2e-2, f"compute-bound: {flops / 1e9:.1f} GFLOP, {tflops:.0f} TFLOP/s = "
         f"{tflops / 2500:.2f} of the 2.5 PFLOP/s bf16 MFMA peak; max abs error vs oracle on "
         f"the sample {err:.2e} (tolerance 2e-2)")
    del kc, vc, q, p_args

    # -- Qwen3-8B verify-step pieces: batch 64, 64-node trees, ctx 2048
    B, T, Hkv, D, L = 64, 64, 8, 128, 36
    rng = np.random.default_rng(args.seed + 3)
    vb = VerifyBatch([2048] * B, [random_tree(T, 8, rng) for _ in range(B)], 256, rng)
    N = B * T
    log("store_kvcache")
    g = torch.Generator().manual_seed(args.seed + 3)
    kk = torch.randn(N, Hkv, D, generator=g).to(torch.bfloat16)
    vv = torch.randn(N, Hkv, D, generator=g).to(torch.bfloat16)
    kcd = torch.zeros(vb.num_blocks, 256, Hkv, D, dtype=torch.bfloat16, device=dev)
    vcd = torch.zeros_like(kcd)
    slots = t(vb.slot_mapping)
    kkd, vvd = kk.to(dev), vv.to(dev)
    us = gpu_us(lambda: store_kvcache(kkd, vvd, kcd, vcd, slots), _C.TIMER_STORE_KV)
    kc_np = np.zeros((vb.num_blocks, 256, Hkv, D), np.uint16)
    vc_np = np.zeros_like(kc_np)
    kk_np, vv_np = kk.view(torch.int16).numpy().view(np.uint16), vv.view(torch.int16).numpy().view(np.uint16)
    cus, _ = cpu_us(lambda: okv.store_kvcache(kk_np, vv_np, kc_np, vc_np, vb.slot_mapping))
    ok = (np.array_equal(kcd.view(torch.int16).cpu().numpy().view(np.uint16), kc_np)
          and np.array_equal(vcd.view(torch.int16).cpu().numpy().view(np.uint16), vc_np))
    emit("store_kvcache", "4096 tree rows (64 x 64), 8 KV heads, d 128, bf16", us,
         float(N * Hkv * D * 2 * 2 * 2), cus, "the whole input", ok)
    del kcd, vcd

    log("kv_compact (worst case)")
    kc36 = torch.empty(L, vb.num_blocks, 256, Hkv, D, dtype=torch.bfloat16, device=dev)
    vc36 = torch.empty_like(kc36)
    path = torch.zeros(B, 9, dtype=torch.int32)
    path[:, 1:] = torch.arange(1, 9, dtype=torch.int32) * 7  # 8 accepted nodes, path[d] >= d
    acc = torch.full((B,), 8, dtype=torch.int32)
    bt, ctx = t(vb.bt), t(vb.ctx)
    pd, ad = path.to(dev), acc.to(dev)
    us = gpu_us(lambda: kv_compact(kc36, vc36, bt, ctx, pd, ad), _C.TIMER_KV_COMPACT, iters=10)
    # oracle on 2 of the 36 layers (bit patterns copied from the GPU caches)
    k2 = kc36[:2].view(torch.int16).cpu().numpy().view(np.uint16).copy()
    v2 = vc36[:2].view(torch.int16).cpu().numpy().view(np.uint16).copy()
    kv_compact(kc36, vc36, bt, ctx, pd, ad)
    cus, _ = cpu_us(lambda: okv.kv_compact(k2, v2, vb.bt, vb.ctx, path.numpy(), acc.numpy(), 256))
    ok = (np.array_equal(kc36[:2].view(torch.int16).cpu().numpy().view(np.uint16), k2)
          and np.array_equal(vc36[:2].view(torch.int16).cpu().numpy().view(np.uint16), v2))
    emit("kv_compact", "36 layers, 64 sequences x 8 accepted rows (worst case), 8 KV heads, d 128",
         us, float(B * 8 * L * 4 * Hkv * D * 2), cus * L / 2, "2 of 36 layers, scaled", ok)
    del kc36, vc36

    log("softmax, rejection walk, top-k")
    g = torch.Generator(device=dev).manual_seed(args.seed + 4)
    logits = (torch.randn(N, V, device=dev, generator=g) * 2).to(torch.bfloat16)
    temps = torch.full((N,), 0.8, device=dev)
    us = gpu_us(lambda: temperature_softmax(logits, temps), _C.TIMER_SOFTMAX)
    probs = temperature_softmax(logits, temps)
    ns = 64
    lg = logits[:ns].float().cpu().numpy()
    cus, ref = cpu_us(lambda: osamp.temperature_softmax(lg, np.full(ns, 0.8, np.float32)))
    ok = bool(np.allclose(probs[:ns].cpu().numpy(), ref, rtol=1e-5, atol=1e-35))
    emit("temperature_softmax", f"[4096, {V}] bf16 -> fp32, T = 0.8", us, float(N * V * 6),
         cus * N / ns, f"{ns} of {N} rows, scaled", ok)

    Pt = probs.view(B, T, V)
    Qt = torch.softmax(torch.randn(B, T, V, device=dev, generator=g) * 2 / 0.8, -1)
    parents = torch.from_numpy(np.stack(vb.parents)).to(dev)
    toks = torch.zeros(B, T, dtype=torch.int32, device=dev)
    child = torch.arange(1, T, device=dev)
    for b in range(B):
        drawn = torch.multinomial(Qt[b], T, replacement=True, generator=g)
        toks[b, 1:] = drawn[parents[b, 1:].long(), child].int()
    Ut = torch.rand(B, T, device=dev, generator=g)
    Uft = torch.rand(B, device=dev, generator=g)
    us = gpu_us(lambda: rejection_sample_tree(Pt, Qt, toks, parents, Ut, Uft), _C.TIMER_REJECTION)
    pth, acc, otok, nxt = (x.cpu().numpy() for x in rejection_sample_tree(Pt, Qt, toks, parents, Ut, Uft))
    ns = 4
    Pn, Qn = Pt[:ns].cpu().numpy(), Qt[:ns].cpu().numpy()
    cus, ref = cpu_us(lambda: osamp.rejection_sample_tree(
        Pn, Qn, toks[:ns].cpu().numpy(), parents[:ns].cpu().numpy(), Ut[:ns].cpu().numpy(),
        Uft[:ns].cpu().numpy(), np.zeros(ns, bool)))
    ok = all(np.array_equal(a[:ns], np.asarray(r)) for a, r in zip((pth, acc, otok, nxt), ref))
    emit("rejection_sample_tree", f"batch 64, 64-node depth-8 trees, vocab {V}, fp32, stochastic",
         us, None, cus * B / ns, f"{ns} of {B} sequences, scaled", ok,
         f"latency-bound walk: reads only the rows it visits, at most all P and Q rows "
         f"({2 * B * T * V * 4 / 1e6:.0f} MB); mean accepted {float(acc.mean()):.2f}")

    # fused sampler: statistics pass over the logits, then the walk on logits + stats
    rtemps = temps
    us = gpu_us(lambda: softmax_stats(logits, rtemps), _C.TIMER_SOFTMAX)
    st = softmax_stats(logits, rtemps)
    x64 = logits[:ns].float().cpu().numpy().astype(np.float64) * (1.4426950408889634 / 0.8)
    m64 = x64.max(1)
    inv64 = 1.0 / np.exp2(x64 - m64[:, None]).sum(1)
    ok = bool(np.allclose(st[:ns, 0].cpu().numpy(), m64, rtol=1e-5)
              and np.allclose(st[:ns, 1].cpu().numpy(), inv64, rtol=1e-5))
    emit("softmax_stats", f"[4096, {V}] bf16, T = 0.8: row max and 1/sum only", us, float(N * V * 2),
         None, "statistics checked against float64 on 64 rows", ok)
    us = gpu_us(lambda: rejection_sample_tree_logits(logits, rtemps, st, Qt, toks, parents, Ut, Uft),
                _C.TIMER_REJECTION)
    fused = rejection_sample_tree_logits(logits, rtemps, st, Qt, toks, parents, Ut, Uft)
    Pst = softmax_from_stats(logits, rtemps, st).view(B, T, V)
    want = rejection_sample_tree(Pst, Qt, toks, parents, Ut, Uft)
    ok = all(torch.equal(a, b_) for a, b_ in zip(fused, want))
    del Pst
    emit("rejection_sample_tree_logits", f"batch 64, 64-node depth-8 trees, vocab {V}: the walk on "
         f"bf16 logits + row statistics", us, None, None,
         "outputs compared with the walk on the probabilities of the same statistics", ok,
         "latency-bound walk: reads the logits (and Q) rows it visits")

    # the same walk with lazy statistics: no statistics pass, the walk computes the
    # statistics of the rows it visits
    us = gpu_us(lambda: rejection_sample_tree_logits_lazy(logits, rtemps, Qt, toks, parents, Ut,
                                                          Uft), _C.TIMER_REJECTION)
    so = torch.full((N, 2), float("nan"), device=dev)
    lazy = rejection_sample_tree_logits_lazy(logits, rtemps, Qt, toks, parents, Ut, Uft,
                                             stats_out=so)
    vis = ~torch.isnan(so[:, 0])
    st2 = st.clone()
    st2[vis] = so[vis]
    Pst = softmax_from_stats(logits, rtemps, st2).view(B, T, V)
    want = rejection_sample_tree(Pst, Qt, toks, parents, Ut, Uft)
    ok = all(torch.equal(a, b_) for a, b_ in zip(lazy[:4], want))
    del Pst
    emit("rejection_sample_tree_logits_lazy", f"batch 64, 64-node depth-8 trees, vocab {V}: the "
         f"walk on bf16 logits computing the statistics of the rows it visits", us, None, None,
         "outputs compared with the walk on the probabilities of the statistics it reports", ok,
         f"replaces the statistics pass ({int(vis.sum())} of {N} rows visited) plus the walk")

    rows = 2048
    us = gpu_us(lambda: topk_logprobs(logits[:rows], 8), _C.TIMER_TOPK)
    lp, tk = topk_logprobs(logits[:rows], 8)
    ns = 16
    lg = logits[:ns].float().cpu().numpy()
    cus, (rtok, rlp) = cpu_us(lambda: odraft.topk_logprobs(lg, 8))
    ok = (np.array_equal(tk[:ns].cpu().numpy(), rtok)
          and bool(np.all(np.abs(lp[:ns].cpu().numpy() - rlp) <= 2e-5 + 1e-6 * np.abs(rlp))))
    emit("topk_logprobs", f"[{rows}, {V}] bf16, k = 8", us, float(rows * V * 2), cus * rows / ns,
         f"{ns} of {rows} rows, scaled", ok)


def parse_socket_power(text):
    """Socket power (W) from `amd-smi metric -p --json` output, or None."""
    import re
    m = re.search(r'"socket_power"\s*:\s*\{[^}]*"value"\s*:\s*([0-9.]+)', text)
    return float(m.group(1)) if m else None


def parse_sclk(text):
    """Shader clock (MHz) from `rocm-smi --showclocks --json` output (which may start
    with a warning line), or None."""
    import re
    m = re.search(r'"sclk clock speed:"\s*:\s*"\((\d+)Mhz\)"', text)
    return float(m.group(1)) if m else None


def parse_power_cap(text):
    """Power cap (W) from `rocm-smi --showmaxpower --json` output, or None."""
    import re
    m = re.search(r'"Max Graphics Package Power \(W\)"\s*:\s*"([0-9.]+)"', text)
    return float(m.group(1)) if m else None


def tool_output(*cmd):
    """stdout of a system tool, or "" when it is missing or fails to answer."""
    import subprocess
    try:
        return subprocess.run(list(cmd), capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        return ""


def smi_reading():
    """One reading of the socket power (W, `amd-smi metric -p`) and the shader clock (MHz,
    `rocm-smi --showclocks`); None for a value the tools do not report."""
    return (parse_socket_power(tool_output("amd-smi", "metric", "-p", "--json")),
            parse_sclk(tool_output("rocm-smi", "--showclocks", "--json")))


def power_cap_w():
    """The board's power cap (W) from `rocm-smi --showmaxpower`, or None."""
    return parse_power_cap(tool_output("rocm-smi", "--showmaxpower", "--json"))


def powered_run(torch, fn, secs, batch=20):
    """Call fn back to back for about secs seconds (synchronising every `batch` calls)
    while a thread samples power and clock every ~0.2 s.  Returns (GPU µs per call from
    CUDA events, power readings, clock readings); the first two readings, taken while
    the part ramps up, are dropped."""
    import threading
    samples, stop = [], threading.Event()

    def poll():
        while not stop.is_set():
            samples.append(smi_reading())
            time.sleep(0.2)

    for _ in range(batch):
        fn()
    torch.cuda.synchronize()
    th = threading.Thread(target=poll)
    calls = 0
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    th.start()
    e0.record()
    t0 = time.time()
    while time.time() - t0 < secs:
        for _ in range(batch):
            fn()
        calls += batch
        torch.cuda.synchronize()
    e1.record()
    torch.cuda.synchronize()
    stop.set()
    th.join()
    body = samples[2:] if len(samples) > 4 else samples
    return (e0.elapsed_time(e1) * 1e3 / calls, [p for p, _ in body if p is not None],
            [c for _, c in body if c is not None])


def run_power(args):
    """Power and clock under the verify-step attention layer, causal prefill, a bf16 GEMM
    and a device copy, each run back to back for --power-secs seconds; one JSON line per
    load and one with the energy budget of the attention layer at the power cap.

    The budget: at the cap, a launch of t us may spend (cap - idle) * t above idle, so
    0.60 of the 8 TB/s roofline (t = algorithmic bytes / 4.8 TB/s) allows that much
    energy per launch.  Against it stand the energy the layer spends now, (measured
    power - idle) * measured time, and its HBM share at the copy's energy per byte; the
    rest, per MFMA FLOP executed, is compared with the GEMM's energy per FLOP (which
    includes the GEMM's own LDS and VALU work)."""
    import threading
    import numpy as np
    import torch
    from nanovllm import _C
    from nanovllm.layers.attention import tree_attention
    from nanovllm.spec.tree import chain_parents, random_tree
    from nanovllm.utils.synthetic import VerifyBatch

    _C.lib()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(args.seed)
    D = 128

    def stat(a):
        return {"mean": float(np.mean(a)), "min": float(np.min(a)), "max": float(np.max(a)),
                "n": len(a)} if a else None

    def attention_load(vb, Hq, Hkv, T, masked):
        kc = torch.randn(vb.num_blocks, 256, Hkv, D, device=dev, generator=g).to(torch.bfloat16)
        vc = torch.randn(vb.num_blocks, 256, Hkv, D, device=dev, generator=g).to(torch.bfloat16)
        N = int(vb.cu_q[-1])
        q = torch.randn(N, Hq, D, device=dev, generator=g).to(torch.bfloat16)
        t = lambda a, dt=torch.int32: torch.from_numpy(np.ascontiguousarray(a)).to(dev, dt)  # noqa: E731
        a_args = (q, kc, vc, t(vb.bt), t(vb.cu_q), t(vb.context_lens), D ** -0.5,
                  t(vb.masks, torch.int64) if masked else None, T, int(vb.context_lens.max()))
        out = torch.empty_like(q)
        if masked:  # MFMA FLOPs executed: every q row against every key of its 64-key chunks
            chunks = np.ceil(vb.context_lens / 64.0) * 64.0
            flops = 4.0 * Hq * D * float((vb.qlens * chunks).sum())
        else:  # causal: the FLOPs of the visible keys
            ql, cl = vb.qlens.astype(np.float64), vb.context_lens.astype(np.float64)
            flops = 4.0 * Hq * D * float(((cl - ql) * ql + ql * (ql + 1) / 2).sum())
        nbytes = float(vb.context_lens.sum()) * Hkv * D * 2 * 2 + 2.0 * N * Hq * D * 2
        return (lambda: tree_attention(*a_args, out=out)), flops, nbytes

    cap = power_cap_w()
    # idle: no launches
    samples, stop = [], threading.Event()

    def poll():
        while not stop.is_set():
            samples.append(smi_reading())
            time.sleep(0.2)

    th = threading.Thread(target=poll)
    th.start()
    time.sleep(2.0)
    stop.set()
    th.join()
    idle_w = [p for p, _ in samples if p is not None]
    idle = float(np.mean(idle_w)) if idle_w else None
    print(json.dumps({"workload": "power", "load": "idle", "power_w": stat(idle_w),
                      "sclk_mhz": stat([c for _, c in samples if c is not None]),
                      "power_cap_w": cap}), flush=True)

    rng = np.random.default_rng(args.seed)
    B, T = 64, 64
    vb4 = VerifyBatch([2048] * B, [random_tree(T, 8, rng) for _ in range(B)], 256, rng)
    vbp = VerifyBatch([0] * 4, [chain_parents(2048)] * 4, 256, rng)
    M = 8192
    A = torch.randn(M, M, device=dev, generator=g).to(torch.bfloat16)
    Bm = torch.randn(M, M, device=dev, generator=g).to(torch.bfloat16)
    C = torch.empty(M, M, device=dev, dtype=torch.bfloat16)
    src = torch.randint(0, 255, (1 << 30,), device=dev, dtype=torch.uint8, generator=g)
    dst = torch.empty_like(src)
    att4, f4, b4 = attention_load(vb4, 32, 8, T, True)
    attp, fp, bp = attention_load(vbp, 32, 8, 2048, False)
    loads = [
        ("tree attention, verify-step layer: 64 sequences x 64-node depth-8 trees, ctx 2048, "
         "32/8 heads", att4, f4, b4),
        ("tree attention, causal prefill: 4 prompts of 2048 tokens, 32/8 heads", attp, fp, bp),
        ("bf16 GEMM 8192 x 8192 x 8192 (torch.mm)", lambda: torch.mm(A, Bm, out=C),
         2.0 * M * M * M, 3.0 * M * M * 2),
        ("device copy, 1 GiB (read + write)", lambda: dst.copy_(src), 0.0, 2.0 * src.numel()),
    ]
    res = {}
    for name, fn, flops, nbytes in loads:
        us, pw, ck = powered_run(torch, fn, args.power_secs)
        p = float(np.mean(pw)) if pw else None
        above = (p - idle) * us * 1e-3 if (p is not None and idle is not None) else None  # mJ
        rec = {"workload": "power", "load": name, "us_per_call": us, "power_w": stat(pw),
               "sclk_mhz": stat(ck), "mj_per_call_above_idle": above,
               "tflops": flops / us / 1e6 if flops else None, "gbs": nbytes / us / 1e3}
        res[name] = (us, p, flops, nbytes)
        print(json.dumps(rec), flush=True)

    gemm = res[loads[2][0]]
    copy = res[loads[3][0]]
    if None in (idle, cap, gemm[1], copy[1]):
        print(json.dumps({"workload": "power", "floor": None,
                          "note": "power readings unavailable"}), flush=True)
        return
    layer = res[loads[0][0]]
    e_flop = (gemm[1] - idle) * gemm[0] * 1e-6 / gemm[2]  # J per FLOP above idle
    e_byte = (copy[1] - idle) * copy[0] * 1e-6 / copy[3]  # J per HBM byte above idle
    e_now = (layer[1] - idle) * layer[0] * 1e-6  # J per launch above idle
    t_target = b4 / (0.60 * HBM_PEAK_GBS * 1e9)  # s
    e_budget = (cap - idle) * t_target
    e_hbm = b4 * e_byte
    print(json.dumps({"workload": "power", "budget": "verify-step attention layer at the cap",
                      "measured_us": layer[0], "measured_power_w": layer[1],
                      "mj_per_launch_now": e_now * 1e3, "target_frac_of_hbm_peak": 0.60,
                      "target_us": t_target * 1e6, "mj_per_launch_allowed_at_cap": e_budget * 1e3,
                      "hbm_mj_at_copy_energy": e_hbm * 1e3, "layer_mfma_flops": f4,
                      "pj_per_flop_rest_now": (e_now - e_hbm) / f4 * 1e12,
                      "pj_per_flop_rest_allowed": (e_budget - e_hbm) / f4 * 1e12,
                      "pj_per_flop_gemm": e_flop * 1e12, "pj_per_byte_copy": e_byte * 1e12}),
          flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "the verify path runs on a single GPU; --gpus must be 1",
                          "n_gpus": args.gpus}), flush=True)
        sys.exit(2)
    if args.workload == "e2e":
        run_e2e(args)
        return
    if args.workload == "kernels":
        run_kernels(args)
        return
    if args.workload == "power":
        run_power(args)
        return
    import torch
    from nanovllm import _C

    dev = torch.device("cuda:0")
    print(f"[bench] building {args.model} verify step: B={args.batch} T={args.tree_nodes} "
          f"depth={args.tree_depth} ctx={args.context}", file=sys.stderr, flush=True)
    step, state = build_step(args, torch, dev)
    for i in range(args.warmup):
        step()
    torch.cuda.synchronize()
    print("[bench] warmup done", file=sys.stderr, flush=True)

    _C.timing_reset()
    _C.timing_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    outs = []
    for i in range(args.steps):
        outs.append(step())
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    accepted = sum(int(o[:, 0].sum()) for o in outs)
    verified = accepted + args.steps * args.batch
    _C.timing_enable(False)
    timers = {k: _C.timing_read(i) for k, i in (
        ("tree_attention", _C.TIMER_TREE_ATTENTION), ("rejection", _C.TIMER_REJECTION),
        ("kv_compact", _C.TIMER_KV_COMPACT), ("store_kvcache", _C.TIMER_STORE_KV))}
    print(f"[bench] timed {args.steps} steps in {elapsed:.3f}s", file=sys.stderr, flush=True)

    vb, cfg = state["vb"], state["cfg"]
    B, T, V = args.batch, args.tree_nodes, cfg.vocab_size
    Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    avg = lambda k: timers[k][0] / max(timers[k][1], 1)
    # tree attention, per launch (one layer): K+V of every cached position read once,
    # q read and o written once.
    attn_bytes = float(vb.context_lens.sum()) * Hkv * D * 2 * 2 + 2.0 * B * T * Hq * D * 2
    attn_ms = avg("tree_attention")
    attn_gbs = attn_bytes / (attn_ms * 1e-3) / 1e9
    traffic, traffic_note = read_pmc_traffic()
    # The sampler is one kernel: the tree walk computes the softmax statistics of each
    # target row it visits (the accepted path of every sequence) and recomputes every
    # probability it reads from the bf16 logits; no statistics pass over all rows and
    # no fp32 probability rows.  Algorithmic bytes: each visited logits row once, plus
    # one bf16 logits row and one fp32 draft row per residual pass (a rejected child);
    # the final draw reads a row the walk has visited.
    parents_np = state["parents"].cpu().numpy()
    rows = [walk_rows(parents_np, o.numpy()) for o in outs]
    visited = sum(float((o[:, 0] + 1).sum()) for o in outs) / len(outs)
    resid = sum(qr for _, qr in rows) / len(rows)
    stats_bytes = visited * V * 2
    walk_bytes = resid * V * (2 + 4)
    walk_ms = avg("rejection")
    sampler_bytes = stats_bytes + walk_bytes
    sampler_gbs = sampler_bytes / (walk_ms * 1e-3) / 1e9
    # The dense form of the sampler reads every fp32 target and draft probability row
    # ([B, T, V] each); its HBM roofline time is what the walk is measured against.
    dense_bytes = 2.0 * B * T * V * 4
    dense_us = dense_bytes / (HBM_PEAK_GBS * 1e9) * 1e6

    out = {
        "metric": METRIC,
        "value": verified / elapsed,
        "unit": "verified tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": elapsed / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, seeded context K/V, trees and draft probs)",
        "config": {"workload": f"{args.model}-shape tree verify step", "batch": B,
                   "tree_nodes": T, "tree_depth": args.tree_depth, "context": args.context,
                   "layers": cfg.num_hidden_layers, "hidden": cfg.hidden_size, "q_heads": Hq,
                   "kv_heads": Hkv, "head_dim": D, "vocab": V, "temperature": args.temperature,
                   "kv_block": 256},
        "mean_accepted_per_step": accepted / (args.steps * B),
        "roofline": {"kernel": "tree_attention", "bound": "hbm", "achieved": attn_gbs,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": attn_gbs / HBM_PEAK_GBS,
                     "traffic": traffic, "algorithmic_bytes": attn_bytes,
                     "avg_launch_us": attn_ms * 1e3, "launches": timers["tree_attention"][1],
                     **({"traffic_note": traffic_note} if traffic_note else {})},
        "sampler": {"path": "one kernel: the tree walk computes the softmax statistics of the "
                            "target rows it visits (exact max, sum in its canonical order) and "
                            "recomputes each probability it reads from the bf16 logits",
                    "walk_avg_us": walk_ms * 1e3,
                    "visited_rows_per_step": visited,
                    "residual_passes_per_step": resid,
                    "stats_bytes_per_step": stats_bytes,
                    "residual_bytes_per_step": walk_bytes,
                    "bytes_per_step": sampler_bytes,
                    "us_per_step": walk_ms * 1e3,
                    "GBs": sampler_gbs, "frac": sampler_gbs / HBM_PEAK_GBS,
                    "dense_bytes_per_step": dense_bytes,
                    "dense_roofline_us": dense_us,
                    "time_vs_dense_roofline": walk_ms * 1e3 / dense_us},
        "kernels_us_per_step": {k: v[0] / args.steps * 1e3 for k, v in timers.items()},
    }
    if args.small_tree_attention:
        # tree attention at the Qwen3-0.6B shape (32 ragged sequences, 32-node trees),
        # timed after the verify steps, with a parity check on a sample
        print("[bench] tree attention, Qwen3-0.6B shape", file=sys.stderr, flush=True)
        c3 = attention_small_tree(torch, dev, args.seed, lambda fn, timer: gpu_launch_us(
            torch, fn, timer), check_seqs=2)
        out["tree_attention_0p6b"] = {k: c3[k] for k in (
            "config", "gpu_us", "algorithmic_bytes", "GBs", "frac", "parity_with_oracle",
            "max_abs_err", "sample")}
        out["tree_attention_0p6b"]["sample"] = "parity: first 2 of 32 sequences vs the oracle"
    if args.calib_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
    if args.parity_seqs > 0:
        print(f"[bench] parity of one more step on {args.parity_seqs} sequences", file=sys.stderr,
              flush=True)
        out["parity"] = integrated_parity(args, torch, state, step, args.parity_seqs)
    if args.cpu_seqs > 0:
        print(f"[bench] cpu baseline on {args.cpu_seqs} sequences", file=sys.stderr, flush=True)
        v, cores, secs = cpu_baseline(args, torch, state, args.cpu_seqs)
        out["cpu_baseline"] = {
            "value": v, "unit": "verified tokens/s", "cores": cores, "kind": "port",
            "sample": f"{args.cpu_seqs} of {B} sequences ({args.cpu_seqs * T} tree rows) through "
                      f"the full verify step on the host: torch-CPU fp32 dense layers + oracle "
                      f"tree attention, softmax, rejection sampling, compaction; {secs:.1f} s",
            **host_info(torch)}
    if args.offline_generate:
        print("[bench] offline generate (Qwen3-0.6B shape, EAGLE-3) in a child process",
              file=sys.stderr, flush=True)
        out["offline_generate"] = offline_generate_record()
    print(json.dumps(out), flush=True)


def offline_generate_record():
    """The offline generate workload (`--workload e2e`: the reference bench.py workload at
    the Qwen3-0.6B shape with EAGLE-3 drafting and HIP graphs) run in a child process, with
    its own engine and memory, summarised for the verify step's JSON line.  A failure is
    recorded in the summary, not raised."""
    import subprocess
    cmd = [sys.executable, os.path.abspath(__file__), "--workload", "e2e"]
    try:
        r = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=900)
    except subprocess.TimeoutExpired:
        return {"error": "timed out after 900 s"}
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    if r.returncode != 0 or not lines:
        return {"error": f"exit code {r.returncode}"}
    d = json.loads(lines[-1])
    return {k: d[k] for k in ("metric", "value", "unit", "elapsed_s", "output_tokens",
                              "mean_accepted_per_verify", "config") if k in d}


if __name__ == "__main__":
    main()
