"""ModelRunner: one process driving one GPU.

Follows the reference's runner (nanovllm/engine/model_runner.py:15-220): paged KV
allocation, host-side packing of the batch, the model forward and sampling, and
HIP-graph capture of the decode / verify steps (model_runner.py:222-257; on by
default, as there).  Tensor-parallel workers and the shm RPC are left out: the path
runs on one GPU.

Speculative decoding (``speculative_method="ngram"``) replaces the decode step by
a verify step:

1. the n-gram drafter proposes up to k tokens per sequence from its history
   (``nvx_ngram_propose`` over the packed histories);
2. each sequence's root (its last token, not yet cached) and draft tokens form a
   chain of T = 1 + max draft length rows at positions ctx .. ctx+T-1; their K/V
   are stored first and attended with the chain mask (``nvx_tree_attention``);
3. the target rows are softmaxed at each sequence's temperature and verified
   (``nvx_rejection_sample_tree``; delta mode: n-gram drafts are deterministic
   proposals); greedy sequences accept while the draft matches the argmax;
4. the accepted tokens plus one recovered/bonus token go back to the scheduler.
A chain's accepted path is already contiguous, so no compaction is needed.

``speculative_method="eagle3"`` drafts with a one-layer EAGLE-3 head
(nanovllm/models/eagle3.py) fed by the target's residual stream at three layers:
the head catches up on every prefill chunk and on every verify step's accepted
rows, expands a top-k tree (nanovllm/spec/eagle3.py), and the target verifies the
tree (delta mode); the accepted path's target KV rows are then compacted
(``nvx_kv_compact``).
"""
import glob
import os

import numpy as np
import torch

from nanovllm.config import Config
from nanovllm.engine.sequence import Sequence
from nanovllm.layers.sampler import RejectionSampler, Sampler, topk_logprobs
from nanovllm.models.eagle3 import Eagle3DraftModel, eagle3_has_qk_norm, load_eagle3_head
from nanovllm.models.qwen3 import Qwen3ForCausalLM, random_init_
from nanovllm.spec.eagle3 import expand_tree, tree_depths, tree_masks
from nanovllm.spec.kv_compact import kv_compact
from nanovllm.spec.ngram import NgramProposer
from nanovllm.spec.tree import ancestor_masks, chain_parents
from nanovllm.utils.context import get_context, reset_context, set_context
from nanovllm.utils.loader import load_checkpoint


def _safetensors(path):
    return sorted(glob.glob(os.path.join(path, "*.safetensors"))) if path and os.path.isdir(path) else []


def _pinned(values, dtype):
    return torch.tensor(values, dtype=dtype, pin_memory=True).cuda(non_blocking=True)


class DraftStates:
    """EAGLE-3 root states resident on the device, one row per sequence: the feature
    the next tree grows from [H], its top-k target tokens [k] and their log-probs [k].
    A verify step gathers its batch's rows with one index and writes them back with
    one index copy, instead of a Python tuple of tensor views per sequence."""

    def __init__(self):
        self.row = {}    # seq_id -> row
        self.free = []
        self.used = 0    # rows handed out so far (free ones included)
        self.feat = self.tok = self.lp = None

    def __len__(self):
        return len(self.row)

    def __contains__(self, seq_id):
        return seq_id in self.row

    def rows(self, seq_ids, create=False):
        """Device int64 rows of the given sequences (new rows for unseen ids if create)."""
        out = []
        for sid in seq_ids:
            r = self.row.get(sid)
            if r is None:
                if not create:
                    raise KeyError(f"no draft state for sequence {sid}")
                if self.free:
                    r = self.free.pop()
                else:
                    r, self.used = self.used, self.used + 1
                self.row[sid] = r
            out.append(r)
        return _pinned(out, torch.int64)

    def get(self, rows):
        return self.feat[rows], self.tok[rows], self.lp[rows]

    def put(self, rows, feat, tok, lp):
        if self.feat is None or self.feat.shape[0] < self.used:
            cap = max(2 * (0 if self.feat is None else self.feat.shape[0]), self.used, 64)
            grown = [torch.empty((cap,) + t.shape[1:], dtype=t.dtype, device=t.device)
                     for t in (feat, tok, lp)]
            if self.feat is not None:
                n = self.feat.shape[0]
                for g, old in zip(grown, (self.feat, self.tok, self.lp)):
                    g[:n] = old
            self.feat, self.tok, self.lp = grown
        self.feat.index_copy_(0, rows, feat)
        self.tok.index_copy_(0, rows, tok)
        self.lp.index_copy_(0, rows, lp)

    def drop(self, seq_id):
        r = self.row.pop(seq_id, None)
        if r is not None:
            self.free.append(r)


class ModelRunner:

    def __init__(self, config: Config, rank: int = 0, event=None):
        self.config = config
        hf_config = config.hf_config
        self.block_size = config.kvcache_block_size
        self.enforce_eager = config.enforce_eager
        self.world_size = 1
        self.rank = rank
        torch.cuda.set_device(rank)
        default_dtype = torch.get_default_dtype()
        torch.set_default_dtype(getattr(hf_config, "dtype", None) or torch.bfloat16)
        torch.set_default_device("cuda")
        self.model = Qwen3ForCausalLM(hf_config)
        self.load_or_init(config.model)
        self.draft = None
        if config.speculative_method == "eagle3":
            self.draft = Eagle3DraftModel(hf_config, draft_vocab=self._draft_vocab(config),
                                          qk_norm=eagle3_has_qk_norm(_safetensors(config.eagle_model)))
            self.draft.bind_target(self.model)
            self.load_or_init_draft(config.eagle_model)
            self.draft_states = DraftStates()
        self.sampler = Sampler()
        self.rejection = RejectionSampler()
        self.allocate_kv_cache()
        self.graphs = {}
        self.eagle_graphs = {}
        self.catchup_graphs = {}
        if not self.enforce_eager:
            self.capture_cudagraph()
        # None, not "cpu": a device context left installed routes every later torch call
        # through a Python TorchFunctionMode (the default device is the CPU either way).
        torch.set_default_device(None)
        torch.set_default_dtype(default_dtype)
        self.proposer = None
        if config.speculative_method == "ngram":
            self.proposer = NgramProposer(config.ngram_max, config.ngram_min,
                                          config.num_speculative_tokens,
                                          capacity=config.max_model_len + config.verify_lookahead)
        self.gen = torch.Generator(device="cuda").manual_seed(config.seed)
        self._chains = {}  # T -> chain parents and masks on the device
        # verify-step statistics: steps per sequence and histogram of accepted draft tokens
        self.spec_stats = {"verify_rows": 0, "accepted": 0, "accepted_hist": {}}

    def load_or_init(self, path):
        files = _safetensors(path)
        if not files:
            random_init_(self.model, seed=self.config.seed)
            return
        load_checkpoint(self.model, files, ignore=(r".*rotary_emb\.inv_freq",))

    @staticmethod
    def _draft_vocab(config):
        """Draft-head vocabulary: the checkpoint's draft_vocab_size, else the config's."""
        path = os.path.join(config.eagle_model, "config.json") if config.eagle_model else ""
        if path and os.path.isfile(path):
            import json
            with open(path) as f:
                n = json.load(f).get("draft_vocab_size")
            if n:
                return int(n)
        return config.eagle_draft_vocab or None

    def load_or_init_draft(self, path):
        files = _safetensors(path)
        if not files:
            random_init_(self.draft, seed=self.config.seed + 1)
            return
        load_eagle3_head(self.draft, files)

    def drop_draft_state(self, seq_id):
        if self.draft is not None:
            self.draft_states.drop(seq_id)
        if self.proposer is not None:
            self.proposer.drop(seq_id)

    def exit(self):
        torch.cuda.synchronize()

    def call(self, method_name, *args):
        return getattr(self, method_name)(*args)

    def allocate_kv_cache(self):
        config = self.config
        hf = config.hf_config
        Hkv = hf.num_key_value_heads
        D = getattr(hf, "head_dim", hf.hidden_size // hf.num_attention_heads)
        dtype = torch.get_default_dtype()
        layers = hf.num_hidden_layers + (1 if self.draft is not None else 0)
        block_bytes = 2 * layers * self.block_size * Hkv * D * dtype.itemsize
        if config.num_kvcache_blocks <= 0:
            free, total = torch.cuda.mem_get_info()
            reserve = 8 << 30  # activations, logits and fp32 probabilities of a step
            config.num_kvcache_blocks = int(free * config.gpu_memory_utilization - reserve) // block_bytes
        assert config.num_kvcache_blocks > 0
        self.kv_cache = torch.empty(2, hf.num_hidden_layers, config.num_kvcache_blocks,
                                    self.block_size, Hkv, D)
        for l, attn in enumerate(self.model.attention_layers()):
            attn.k_cache = self.kv_cache[0, l]
            attn.v_cache = self.kv_cache[1, l]
        if self.draft is not None:
            # the draft head's one layer, paged with the target's block tables
            self.draft_kv_cache = torch.empty(2, config.num_kvcache_blocks, self.block_size, Hkv, D)
            attn = self.draft.attention_layers()[0]
            attn.k_cache, attn.v_cache = self.draft_kv_cache[0], self.draft_kv_cache[1]

    def prepare_block_tables(self, seqs: list[Sequence]):
        max_len = max(len(seq.block_table) for seq in seqs)
        block_tables = [seq.block_table + [-1] * (max_len - len(seq.block_table)) for seq in seqs]
        return _pinned(block_tables, torch.int32)

    def prepare_prefill(self, seqs: list[Sequence]):
        input_ids, positions, slot_mapping, ctx_lens = [], [], [], []
        cu_seqlens_q, cu_seqlens_k = [0], [0]
        max_seqlen_q = max_seqlen_k = 0
        for seq in seqs:
            start = seq.num_cached_tokens
            end = start + seq.num_scheduled_tokens
            input_ids.extend(seq[start:end])
            positions.extend(range(start, end))
            cu_seqlens_q.append(cu_seqlens_q[-1] + end - start)
            cu_seqlens_k.append(cu_seqlens_k[-1] + end)
            max_seqlen_q = max(end - start, max_seqlen_q)
            max_seqlen_k = max(end, max_seqlen_k)
            ctx_lens.append(end)
            bt = np.asarray(seq.block_table, np.int64)
            pos = np.arange(start, end)
            slot_mapping.extend((bt[pos // self.block_size] * self.block_size
                                 + pos % self.block_size).tolist())
        set_context(True, _pinned(cu_seqlens_q, torch.int32), _pinned(cu_seqlens_k, torch.int32),
                    max_seqlen_q, max_seqlen_k, _pinned(slot_mapping, torch.int32),
                    _pinned(ctx_lens, torch.int32), self.prepare_block_tables(seqs))
        return _pinned(input_ids, torch.int64), _pinned(positions, torch.int64)

    def prepare_decode(self, seqs: list[Sequence], drafts=None):
        """Rows per sequence: the root (last token) then its draft tokens (a chain),
        padded to the longest draft (to the captured graph's rows when graphs are on)."""
        T = 1 + (max(len(d) for d in drafts) if drafts else 0)
        if self.graphs and len(seqs) <= self.graph_bs[-1]:
            T = min(t for t in self.graph_vars if t >= T)
        B = len(seqs)
        ctx = [len(seq) - 1 for seq in seqs]
        self._check_pages(seqs, ctx, T)
        if T == 1:
            input_ids = [seq.last_token for seq in seqs]
            num_nodes = [1] * B
        else:
            ids = np.zeros((B, T), dtype=np.int64)
            num_nodes = []
            for i, (seq, d) in enumerate(zip(seqs, drafts)):
                ids[i, 0] = seq.last_token
                ids[i, 1:1 + len(d)] = d
                num_nodes.append(1 + len(d))
            input_ids = ids.reshape(-1).tolist()
        # positions ctx .. ctx+T-1 of each sequence, their cache slots and the chain
        # masks are built on the device
        block_tables = self.prepare_block_tables(seqs)
        ctx_d = _pinned(ctx, torch.int64)
        positions = (ctx_d.unsqueeze(1) + torch.arange(T, device="cuda")).reshape(-1)
        set_context(False, cu_seqlens_q=torch.arange(0, B * T + 1, T, dtype=torch.int32, device="cuda"),
                    max_seqlen_q=T, slot_mapping=self._slot_grid(block_tables, ctx_d, T).reshape(-1),
                    context_lens=(ctx_d + T).to(torch.int32), block_tables=block_tables,
                    tree_mask=None if T == 1 else self._chain(T)[1].repeat(B),
                    max_context_len=max(ctx) + T)
        return (_pinned(input_ids, torch.int64), positions, T, _pinned(num_nodes, torch.int32))

    def _chain(self, T):
        """Device (parents int32 [T], ancestor masks int64 [T]) of a T-node chain."""
        c = self._chains.get(T)
        if c is None:
            par = chain_parents(T)
            c = (torch.from_numpy(par).cuda(), torch.from_numpy(ancestor_masks(par)).cuda())
            self._chains[T] = c
        return c

    def prepare_sample(self, seqs: list[Sequence]):
        return _pinned([seq.temperature for seq in seqs], torch.float32)

    @torch.inference_mode()
    def run_model(self, input_ids, positions, is_prefill):
        if not is_prefill and self._graph_fits(input_ids.numel()):
            return self.model.compute_logits(self.replay_graph(input_ids, positions))
        hidden = self.model(input_ids, positions)
        if is_prefill:  # logits of each sequence's last scheduled token only
            cu = get_context().cu_seqlens_q
            hidden = hidden[cu[1:].long() - 1]
        return self.model.compute_logits(hidden)

    # ------------------------------------------------------------ HIP graphs ----
    # Verify / decode steps replay a captured target forward (reference
    # model_runner.py:222-257, there for q_len = 1).  A graph covers bs sequences of
    # T rows each (T = 1 or the longest verify chain, a step using the smallest that
    # fits its drafts), with static input and context buffers per T; the attention
    # launch is sized for max_model_len, so any context up to it fits.  Batches are
    # padded to the next captured size with empty sequences (context 0, slot -1:
    # nothing stored, output rows 0).  The LM head and the sampler run outside the
    # graph.  With EAGLE-3 one graph per batch size holds the whole step up to the
    # logits: the draft tree expansion, the verify rows built from it on the device,
    # and the target's tree verify with the aux residual streams the draft head fuses;
    # the draft catch-up is captured per batch size too.

    def _graph_rows(self):
        """Rows per sequence of the captured graphs: the EAGLE-3 tree, or both a plain
        decode row and the longest verify chain (a step replays the smallest that fits)."""
        cfg = self.config
        if cfg.speculative_method == "eagle3":
            return [1 + cfg.num_speculative_tokens]
        return sorted({1, cfg.verify_lookahead})

    def _graph_fits(self, rows):
        ctx = get_context()
        if not self.graphs or ctx.context_lens is None:
            return False
        bs = ctx.context_lens.numel()
        return 0 < bs <= self.graph_bs[-1] and rows % bs == 0 and rows // bs in self.graph_vars

    @torch.inference_mode()
    def capture_cudagraph(self):
        cfg = self.config
        max_bs = min(cfg.max_num_seqs, 512)
        self.graph_bs = [b for b in [1, 2, 4, 8] + list(range(16, max_bs + 1, 16)) if b <= max_bs]
        self.graph_vars = {}
        pool = None
        if self.draft is None:
            for T in sorted(self._graph_rows(), reverse=True):
                pool = self._capture_rows(T, max_bs, pool)
        else:
            T = 1 + cfg.num_speculative_tokens
            self._graph_buffers(T, max_bs)
            pool = self._capture_eagle_steps(max_bs, pool)
            self._capture_catch_up(max_bs, pool)

    def _capture_eagle_steps(self, max_bs, pool):
        """One graph per captured batch size for the EAGLE-3 step up to the target's
        hidden states: the draft tree expansion (every draft level, its top-k and the
        tree selection) over static root states, then the verify rows built from the
        tree on the device (tokens, positions ctx + depth, slots ctx + i, ancestor
        masks), then the target's tree verify with its aux residual streams.  Inputs
        are static buffers the step fills (root states, root tokens, cached lengths,
        block tables, a valid flag per sequence); padding sequences have no pages,
        context 0 and slot -1.  Both attention launches are sized for max_model_len."""
        cfg = self.config
        k, T = cfg.eagle_topk, 1 + cfg.num_speculative_tokens
        H = cfg.hf_config.hidden_size
        gv = self.graph_vars[T]
        # root token, cached length and valid flag per sequence share one buffer, so a
        # step fills them with one copy
        meta = torch.zeros(max_bs, 3, dtype=torch.int64)
        dg = dict(
            root_feat=torch.zeros(max_bs, H),
            root_tok=torch.zeros(max_bs, k, dtype=torch.int64),
            root_lp=torch.zeros(max_bs, k, dtype=torch.float32),
            meta=meta, roots=meta[:, 0], ctx=meta[:, 1], valid=meta[:, 2],
            block_tables=torch.full((max_bs, gv["max_blocks"]), -1, dtype=torch.int32),
            tokens=torch.zeros(max_bs, T - 1, dtype=torch.int64),
            parents=torch.zeros(max_bs, T, dtype=torch.int64),
            depths=torch.zeros(max_bs, T, dtype=torch.int64),
            masks=torch.zeros(max_bs, T, dtype=torch.int64),
            vtok=torch.zeros(max_bs, T, dtype=torch.int32),
            vpar=torch.zeros(max_bs, T, dtype=torch.int32),
        )
        self.draft_graph_vars = dg
        # pinned host staging: the step's meta and block tables, and the read-back of
        # the accepted lengths and tokens
        host = dict(device="cpu", pin_memory=True)
        self._pin_meta = torch.zeros(max_bs, 3, dtype=torch.int64, **host)
        self._pin_bt = torch.full((max_bs, gv["max_blocks"]), -1, dtype=torch.int32, **host)
        self._pin_acc = torch.zeros(max_bs, dtype=torch.int32, **host)
        self._pin_out = torch.zeros(max_bs, T, dtype=torch.int32, **host)
        for bs in reversed(self.graph_bs):
            def step():
                ctx_d, bt = dg["ctx"][:bs], dg["block_tables"][:bs]
                outs = self._expand_draft_tree(dg["root_tok"][:bs], dg["root_lp"][:bs],
                                               dg["root_feat"][:bs], ctx_d, bt, cfg.max_model_len)
                for name, t in zip(("tokens", "parents", "depths", "masks"), outs):
                    dg[name][:bs] = t
                tree_tok, parents, depths, masks = outs
                tokens = torch.cat([dg["roots"][:bs].unsqueeze(1), tree_tok], dim=1)
                dg["vtok"][:bs] = tokens
                dg["vpar"][:bs] = parents
                h, a = self._verify_tree(tokens, depths, masks, ctx_d, bt, dg["valid"][:bs] != 0,
                                         cfg.max_model_len)
                gv["outputs"][:bs * T] = h
                gv["aux"][:bs * T] = a

            step()  # warmup
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool):
                step()
            if pool is None:
                pool = graph.pool()
            self.eagle_graphs[bs] = graph
            torch.cuda.synchronize()
        return pool

    def _verify_tree(self, tokens, depths, masks, ctx_d, block_tables, valid, max_ctx):
        """The target's tree verify from device tensors only (capturable): tokens, depths,
        masks [B, T]; node i at position ctx + depth(i), stored at ctx + i; invalid
        (padding) sequences have context 0.  Returns (hidden [B*T, H], aux)."""
        B, T = tokens.shape
        dev = tokens.device
        positions = (ctx_d.unsqueeze(1) + depths).reshape(-1)
        slot_mapping = self._slot_grid(block_tables, ctx_d, T).reshape(-1)
        context_lens = torch.where(valid, ctx_d + T, 0).to(torch.int32)
        set_context(False, cu_seqlens_q=torch.arange(0, B * T + 1, T, dtype=torch.int32, device=dev),
                    max_seqlen_q=T, slot_mapping=slot_mapping, context_lens=context_lens,
                    block_tables=block_tables, tree_mask=masks.reshape(-1).contiguous(),
                    max_context_len=max_ctx)
        try:
            return self.model(tokens.reshape(-1), positions, self.draft.aux_layers)
        finally:
            reset_context()

    def _capture_catch_up(self, max_bs, pool):
        cfg = self.config
        k, depth, T = cfg.eagle_topk, cfg.eagle_depth, 1 + cfg.num_speculative_tokens
        H = cfg.hf_config.hidden_size
        dg = self.draft_graph_vars

        # Draft catch-up per batch size: depth + 1 rows per sequence (the longest
        # accepted path plus the bonus token), rows past a sequence's accepted length
        # padded (slot -1, outside every real row's causal window); the target
        # features come from the verify graph's aux buffer.
        D1 = min(depth, T - 1) + 1  # the longest accepted path, plus its bonus token
        gv = self.graph_vars[T]
        cg = dict(
            acc=torch.zeros(max_bs, dtype=torch.int64),
            path=torch.zeros(max_bs, D1, dtype=torch.int64),
            out=torch.zeros(max_bs, D1, dtype=torch.int64),
            feat=torch.zeros(max_bs, H),
            tok=torch.zeros(max_bs, k, dtype=torch.int64),
            lp=torch.zeros(max_bs, k, dtype=torch.float32),
        )
        self.catchup_graph_vars = cg
        for bs in reversed(self.graph_bs):
            def catch_up():
                outs = self._catch_up_padded(cg["acc"][:bs], cg["path"][:bs], cg["out"][:bs],
                                             dg["ctx"][:bs], dg["block_tables"][:bs], gv["aux"],
                                             T, cfg.max_model_len)
                for name, t in zip(("feat", "tok", "lp"), outs):
                    cg[name][:bs] = t

            catch_up()  # warmup
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool):
                catch_up()
            self.catchup_graphs[bs] = graph
            torch.cuda.synchronize()

    def _catch_up_padded(self, acc, path, out_tokens, ctx_d, block_tables, aux, T, max_ctx):
        """The draft catch-up over a fixed depth+1 rows per sequence (device tensors only,
        so it can be captured): row j of sequence b is position ctx_b + j with the accepted
        path's token j and the target feature of tree row path[b, j]; rows j > acc_b are
        padding (no K/V stored, after every real row in the causal order).  Returns the
        next root states (feature, top-k tokens, log-probs) [B, ...]."""
        B, D1 = path.shape
        dev = acc.device
        j = torch.arange(D1, device=dev)
        seq = torch.arange(B, device=dev).unsqueeze(1)
        valid = j.unsqueeze(0) <= acc.unsqueeze(1)
        pos = ctx_d.unsqueeze(1) + j
        slots = torch.where(valid, self._slots_of(block_tables, seq, pos), -1).reshape(-1)
        tree_rows = (seq * T + path.clamp(min=0)).reshape(-1)
        ids = torch.where(valid, out_tokens, 0).reshape(-1)
        set_context(True, torch.arange(0, B * D1 + 1, D1, dtype=torch.int32, device=dev), None,
                    D1, max_ctx, slots, (ctx_d + D1).to(torch.int32), block_tables)
        normed, feats = self.draft(ids, pos.reshape(-1), self.draft.fuse(aux[tree_rows]))
        reset_context()
        return self._draft_state(normed, feats, seq.squeeze(1) * D1 + acc)

    def _graph_buffers(self, T, max_bs):
        """Static buffers of the captured steps with T rows per sequence."""
        cfg, hf = self.config, self.config.hf_config
        aux_layers = self.draft.aux_layers if self.draft is not None else None
        reserve = max(T, cfg.verify_lookahead)  # slots a step may reserve past the context
        max_blocks = (cfg.max_model_len + reserve + self.block_size - 1) // self.block_size
        rows = max_bs * T
        gv = dict(
            rows=rows, T=T, max_blocks=max_blocks,
            input_ids=torch.zeros(rows, dtype=torch.int64),
            positions=torch.zeros(rows, dtype=torch.int64),
            slot_mapping=torch.full((rows,), -1, dtype=torch.int32),
            context_lens=torch.zeros(max_bs, dtype=torch.int32),
            block_tables=torch.full((max_bs, max_blocks), -1, dtype=torch.int32),
            cu_seqlens_q=torch.arange(0, rows + 1, T, dtype=torch.int32),
            tree_mask=torch.from_numpy(np.tile(ancestor_masks(chain_parents(T)), max_bs)).cuda()
            if T > 1 else None,
            outputs=torch.zeros(rows, hf.hidden_size),
            aux=torch.zeros(rows, len(aux_layers) * hf.hidden_size) if aux_layers else None,
        )
        self.graph_vars[T] = gv
        return gv

    def _capture_rows(self, T, max_bs, pool):
        cfg = self.config
        aux_layers = self.draft.aux_layers if self.draft is not None else None
        gv = self._graph_buffers(T, max_bs)
        for bs in reversed(self.graph_bs):
            n = bs * T
            set_context(False, cu_seqlens_q=gv["cu_seqlens_q"][:bs + 1], max_seqlen_q=T,
                        slot_mapping=gv["slot_mapping"][:n], context_lens=gv["context_lens"][:bs],
                        block_tables=gv["block_tables"][:bs],
                        tree_mask=None if T == 1 else gv["tree_mask"][:n],
                        max_context_len=cfg.max_model_len)
            def forward():
                if aux_layers is None:
                    gv["outputs"][:n] = self.model(gv["input_ids"][:n], gv["positions"][:n])
                else:
                    h, a = self.model(gv["input_ids"][:n], gv["positions"][:n], aux_layers)
                    gv["outputs"][:n] = h
                    gv["aux"][:n] = a

            forward()  # warmup
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool):
                forward()
            if pool is None:
                pool = graph.pool()
            self.graphs[(T, bs)] = graph
            torch.cuda.synchronize()
            reset_context()
        return pool

    def replay_graph(self, input_ids, positions):
        ctx = get_context()
        bs = ctx.context_lens.numel()
        n = input_ids.numel()
        if not self._graph_fits(n):
            raise RuntimeError(f"replay_graph: no captured graph for {n} rows of {bs} sequences "
                               f"(rows per sequence {sorted(self.graph_vars)})")
        gv = self.graph_vars[n // bs]
        g = next(b for b in self.graph_bs if b >= bs)
        gv["input_ids"][:n] = input_ids
        gv["positions"][:n] = positions
        gv["slot_mapping"].fill_(-1)
        gv["slot_mapping"][:n] = ctx.slot_mapping
        gv["context_lens"].zero_()
        gv["context_lens"][:bs] = ctx.context_lens
        gv["block_tables"].fill_(-1)
        bt = ctx.block_tables
        gv["block_tables"][:bs, :bt.shape[1]] = bt
        if gv["tree_mask"] is not None:
            gv["tree_mask"][:n] = ctx.tree_mask
        self.graphs[(gv["T"], g)].replay()
        if gv["aux"] is not None:
            return gv["outputs"][:n], gv["aux"][:n]
        return gv["outputs"][:n]

    @torch.inference_mode()
    def run(self, seqs: list[Sequence], is_prefill: bool):
        if self.draft is not None:
            return self.run_eagle_prefill(seqs) if is_prefill else self.run_eagle_verify(seqs)
        if is_prefill:
            input_ids, positions = self.prepare_prefill(seqs)
            temperatures = self.prepare_sample(seqs)
            logits = self.run_model(input_ids, positions, True)
            token_ids = self._sampled(self.sampler(logits, temperatures).tolist())
            reset_context()
            return token_ids
        drafts = (self.proposer.propose_seqs([seq.seq_id for seq in seqs],
                                             [seq.token_ids for seq in seqs])
                  if self.proposer else None)
        input_ids, positions, T, num_nodes = self.prepare_decode(seqs, drafts)
        temperatures = self.prepare_sample(seqs)
        logits = self.run_model(input_ids, positions, False)
        reset_context()
        B = len(seqs)
        if T == 1:
            return [[t] for t in self._sampled(self.sampler(logits, temperatures).tolist())]
        tokens = input_ids.view(B, T).to(torch.int32)
        parents = self._chain(T)[0].repeat(B, 1)
        U, Uf = self._uniforms(B, T)
        _, acc, out_tokens, _ = self.rejection(logits, temperatures, None, tokens, parents, U, Uf,
                                               num_nodes)
        return self._verified_tokens(acc.tolist(), out_tokens.tolist())

    def _uniforms(self, B, T):
        """The walk's uniforms: [B, T] for the acceptance tests, [B] for the final draws."""
        dev = self.gen.device
        return (torch.rand(B, T, device=dev, generator=self.gen),
                torch.rand(B, device=dev, generator=self.gen))

    @staticmethod
    def _sampled(token_ids):
        """Host list of the sampler's tokens; a -1 (a walk whose workgroups failed to
        meet) is refused before it can reach the scheduler or an embedding lookup."""
        if token_ids and min(token_ids) < 0:
            bad = [i for i, t in enumerate(token_ids) if t < 0]
            raise RuntimeError(f"sampler walk failed for {len(bad)} of {len(token_ids)} rows "
                               f"(rows {bad[:8]}{' ...' if len(bad) > 8 else ''})")
        return token_ids

    def _verified_tokens(self, acc, out_tokens):
        """Host lists of the walk's outputs -> each sequence's accepted tokens followed by
        its recovered / bonus token.  A multi-workgroup walk whose workgroups failed to
        meet writes accepted_len = -1 (and -1 tokens); such a step is refused here, before
        anything is counted, handed to the scheduler or used as a draft root."""
        bad = [b for b, a in enumerate(acc) if a < 0]
        if bad:
            raise RuntimeError(
                f"tree rejection walk failed for {len(bad)} of {len(acc)} sequences (batch rows "
                f"{bad[:8]}{' ...' if len(bad) > 8 else ''}): its workgroups did not meet within "
                f"the bounded wait, so this verify step produced no tokens")
        self._count(acc)
        return [out_tokens[b][:acc[b] + 1] for b in range(len(acc))]

    def _count(self, acc):
        st = self.spec_stats
        st["verify_rows"] += len(acc)
        st["accepted"] += sum(acc)
        for a in acc:
            st["accepted_hist"][a] = st["accepted_hist"].get(a, 0) + 1

    # ---------------------------------------------------------------- EAGLE-3 ----

    def _slots_of(self, block_tables, b, pos):
        """Cache slots, int32, of positions pos of sequences b (int64 tensors that
        broadcast together), from the padded block tables (int32 [B, max_blocks]).
        Past the end of a sequence's table the slot is negative (nothing is stored);
        the scheduler reserves the pages of every row a step writes
        (_check_pages)."""
        bs = self.block_size
        idx = (pos // bs).clamp(max=block_tables.shape[1] - 1)
        blk = block_tables[b, idx].to(torch.int64)
        return torch.where(blk >= 0, blk * bs + pos % bs, -1).to(torch.int32)

    def _slot_grid(self, block_tables, start, count):
        """Slots of positions start_b .. start_b + count - 1 of every sequence: [B, count]."""
        B = start.shape[0]
        pos = start.unsqueeze(1) + torch.arange(count, device=start.device)
        return self._slots_of(block_tables, torch.arange(B, device=start.device).unsqueeze(1), pos)

    def _check_pages(self, seqs, ctx, rows):
        for seq, c in zip(seqs, ctx):
            if len(seq.block_table) * self.block_size < c + rows:
                raise RuntimeError(f"sequence {seq.seq_id}: {len(seq.block_table)} pages do not "
                                   f"hold positions {c} .. {c + rows - 1}")

    def _draft_state(self, normed, features, rows):
        """Top-k of the next-token distribution after the given draft rows, and the
        rows' output features (the state the next tree grows from)."""
        lp, tok = topk_logprobs(self.draft.compute_logits(normed[rows]), self.config.eagle_topk)
        return features[rows], self.draft.to_target(tok), lp

    def run_eagle_prefill(self, seqs):
        input_ids, positions = self.prepare_prefill(seqs)
        temperatures = self.prepare_sample(seqs)
        hidden, aux = self.model(input_ids, positions, self.draft.aux_layers)
        cu = get_context().cu_seqlens_q
        last = cu[1:].long() - 1
        token_ids = self._sampled(
            self.sampler(self.model.compute_logits(hidden[last]), temperatures).tolist())
        # Draft catch-up on the chunk: row q takes token q+1 (the sampled token after
        # the prompt's last position) and the target feature at q.  Same attention
        # context as the target's prefill (positions, slots, block tables).
        shifted = []
        for seq, tok in zip(seqs, token_ids):
            start = seq.num_cached_tokens
            end = start + seq.num_scheduled_tokens
            nxt = seq[end] if end < seq.num_tokens else tok
            shifted.extend(seq[start + 1:end] + [nxt])
        normed, feats = self.draft(_pinned(shifted, torch.int64), positions, self.draft.fuse(aux))
        done = [i for i, seq in enumerate(seqs)
                if seq.num_cached_tokens + seq.num_scheduled_tokens == seq.num_tokens]
        if done:
            rows = last[torch.tensor(done, device=last.device)]
            f, tok, lp = self._draft_state(normed, feats, rows)
            st = self.draft_states
            st.put(st.rows([seqs[i].seq_id for i in done], create=True), f, tok, lp)
        reset_context()
        return token_ids

    def _eagle_graphed(self, B):
        return bool(self.eagle_graphs) and B <= self.graph_bs[-1]

    def _replay_eagle_step(self, seqs, rows, ctx, block_tables=None):
        """Fill the captured EAGLE-3 step's static inputs and replay it: the root states
        of the sequences' DraftStates rows (gathered on the device), and root tokens,
        cached lengths, valid flags and block tables from pinned host staging (one copy
        each); the batch is padded to the next captured size with empty sequences.  The
        tree lands in draft_graph_vars, the target's hidden states and aux streams in
        graph_vars[T].  block_tables: the sequences' padded device tables (only their
        width is used when given; the staging is built from the sequences)."""
        B = len(seqs)
        g = next(b for b in self.graph_bs if b >= B)
        dg = self.draft_graph_vars
        st = self.draft_states
        for name, src in (("root_feat", st.feat), ("root_tok", st.tok), ("root_lp", st.lp)):
            torch.index_select(src, 0, rows, out=dg[name][:B])
            if g > B:
                dg[name][B:g].zero_()
        meta = self._pin_meta.numpy()
        meta[:g] = 0
        meta[:B, 0] = [seq.last_token for seq in seqs]
        meta[:B, 1] = ctx
        meta[:B, 2] = 1
        bt = self._pin_bt.numpy()
        bt[:g] = -1
        for i, seq in enumerate(seqs):
            bt[i, :len(seq.block_table)] = seq.block_table
        dg["meta"][:g].copy_(self._pin_meta[:g], non_blocking=True)
        dg["block_tables"][:g].copy_(self._pin_bt[:g], non_blocking=True)
        self.eagle_graphs[g].replay()

    def _eagle_tree(self, seqs, ctx, block_tables, rows=None):
        """Expand one draft tree per sequence from its resident root state (rows: the
        sequences' DraftStates rows, looked up when not given).  Returns tokens
        [B, T-1], parents [B, T], node depths [B, T] and ancestor masks [B, T].
        With graphs on and a batch that fits, replays the captured EAGLE-3 step (which
        also runs the target's verify of the tree) and returns copies of its tree."""
        B = len(seqs)
        if rows is None:
            rows = self.draft_states.rows([seq.seq_id for seq in seqs])
        ctx_d = _pinned(ctx, torch.int64)
        if self._eagle_graphed(B):
            self._replay_eagle_step(seqs, rows, ctx)
            dg = self.draft_graph_vars
            return tuple(dg[name][:B].clone() for name in ("tokens", "parents", "depths", "masks"))
        root_feat, root_tok, root_lp = self.draft_states.get(rows)
        return self._expand_draft_tree(root_tok, root_lp, root_feat, ctx_d, block_tables, max(ctx))

    def _expand_draft_tree(self, root_tok, root_lp, root_feat, ctx_d, block_tables, max_ctx):
        """The draft head's levels over device tensors only (no host reads, so it can be
        captured): root top-k [B, k] and feature [B, H], cached lengths [B] and block
        tables; max_ctx bounds every cached length.  The expanded rows' cache slots
        (positions ctx .. ctx + rmax - 1) come from the block tables.  Returns the
        tree (tokens, parents) and its node depths and ancestor masks."""
        cfg = self.config
        k, depth, T = cfg.eagle_topk, cfg.eagle_depth, 1 + cfg.num_speculative_tokens
        B = root_tok.shape[0]
        rmax = k * max(depth - 1, 1)
        row_level = torch.arange(rmax, device="cuda") // k        # position offset of row r
        H = root_feat.shape[-1]
        slots = self._slot_grid(block_tables, ctx_d, rmax)

        def draft_rows(rows_tok, rows_feat, rows_mask, level):
            R = rows_tok.shape[1]
            positions = (ctx_d.unsqueeze(1) + row_level[:R]).reshape(-1)
            set_context(False, cu_seqlens_q=torch.arange(0, B * R + 1, R, dtype=torch.int32,
                                                         device="cuda"),
                        max_seqlen_q=R, slot_mapping=slots[:, :R].reshape(-1).contiguous(),
                        context_lens=(ctx_d + R).to(torch.int32), block_tables=block_tables,
                        tree_mask=rows_mask.reshape(-1).contiguous(), max_context_len=max_ctx + R)
            normed, feats = self.draft(rows_tok.reshape(-1), positions, rows_feat.reshape(B * R, H))
            reset_context()
            last = normed.view(B, R, H)[:, R - k:].reshape(B * k, H)
            lp, tok = topk_logprobs(self.draft.compute_logits(last), k)
            tok = self.draft.to_target(tok)
            return (tok.view(B, k, k), lp.view(B, k, k)), feats.view(B, R, H)[:, R - k:]

        tokens, parents = expand_tree(draft_rows, root_tok, root_lp, root_feat, depth, T)
        return tokens, parents, tree_depths(parents, depth), tree_masks(parents, depth)

    def run_eagle_verify(self, seqs):
        cfg = self.config
        T = 1 + cfg.num_speculative_tokens
        B = len(seqs)
        ctx = [len(seq) - 1 for seq in seqs]
        self._check_pages(seqs, ctx, cfg.verify_lookahead)
        rows = self.draft_states.rows([seq.seq_id for seq in seqs])
        graphed = self._eagle_graphed(B)
        if graphed:
            # one replay: draft tree expansion, verify rows, target verify with aux
            self._replay_eagle_step(seqs, rows, ctx)
            gv, dg = self.graph_vars[T], self.draft_graph_vars
            hidden, aux = gv["outputs"][:B * T], gv["aux"][:B * T]
            tok32, par32 = dg["vtok"][:B], dg["vpar"][:B]
            ctx_d, block_tables = dg["ctx"][:B], dg["block_tables"][:B]
        else:
            block_tables = self.prepare_block_tables(seqs)
            ctx_d = _pinned(ctx, torch.int64)
            tree_tok, parents, depths, masks = self._eagle_tree(seqs, ctx, block_tables, rows)
            # target verify of the trees: node i at position ctx + depth(i), stored at ctx + i
            roots = _pinned([seq.last_token for seq in seqs], torch.int64)
            tokens = torch.cat([roots.unsqueeze(1), tree_tok], dim=1)            # [B, T]
            valid = torch.ones(B, dtype=torch.bool, device="cuda")
            hidden, aux = self._verify_tree(tokens, depths, masks, ctx_d, block_tables, valid,
                                            max(ctx) + T)
            tok32, par32 = tokens.to(torch.int32), parents.to(torch.int32)
        logits = self.model.compute_logits(hidden)
        temperatures = self.prepare_sample(seqs)
        U, Uf = self._uniforms(B, T)
        path, acc, out_tokens, _ = self.rejection(logits, temperatures, None, tok32, par32, U, Uf)
        ctx32 = ctx_d.to(torch.int32)
        # a failed walk row (accepted_len -1) compacts nothing
        kv_compact(self.kv_cache[0], self.kv_cache[1], block_tables, ctx32, path, acc)
        # Draft catch-up: rows ctx .. ctx+a take the accepted tokens then the bonus /
        # recovered token, with the target features of the accepted path's tree rows.
        if graphed and self.catchup_graphs:
            # The read-back is an asynchronous copy into pinned memory with an event
            # behind it; the captured catch-up is queued after it, so the GPU runs the
            # catch-up while the host checks the tokens and schedules the next step.  A
            # failed walk row enters the catch-up with accepted length 0 (clamped on
            # the device, never -1), and the check after the event raises.
            acc_h, out_h = self._pin_acc[:B], self._pin_out[:B]
            acc_h.copy_(acc, non_blocking=True)
            out_h.copy_(out_tokens, non_blocking=True)
            landed = torch.cuda.Event()
            landed.record()
            state = self._replay_catch_up(acc.clamp(min=0), path, out_tokens, ctx_d, block_tables,
                                          staged=True)
            self.draft_states.put(rows, *state)
            landed.synchronize()
            return self._verified_tokens(acc_h.tolist(), out_h.tolist())
        acc_h = acc.tolist()
        result = self._verified_tokens(acc_h, out_tokens.tolist())
        state = self._catch_up_packed(acc, acc_h, path, out_tokens, ctx, ctx_d, block_tables,
                                      aux, T)
        self.draft_states.put(rows, *state)
        return result

    def _replay_catch_up(self, acc, path, out_tokens, ctx_d, block_tables, staged=False):
        """The captured catch-up (batch padded to a captured size); the target features
        are the verify graph's aux rows of this step.  staged: the step's replay already
        filled the cached lengths and block tables.  Returns views of its outputs."""
        B = acc.shape[0]
        g = next(b for b in self.graph_bs if b >= B)
        cg, dg = self.catchup_graph_vars, self.draft_graph_vars
        D1 = cg["path"].shape[1]
        for name, src in (("acc", acc), ("path", path[:, :D1]), ("out", out_tokens[:, :D1])):
            cg[name][:B] = src
            cg[name][B:g].zero_()
        if not staged:
            dg["ctx"].zero_()
            dg["ctx"][:B] = ctx_d
            dg["block_tables"].fill_(-1)
            dg["block_tables"][:B, :block_tables.shape[1]] = block_tables
        self.catchup_graphs[g].replay()
        return cg["feat"][:B], cg["tok"][:B], cg["lp"][:B]

    def _catch_up_packed(self, acc, acc_h, path, out_tokens, ctx, ctx_d, block_tables, aux, T):
        """The eager catch-up over exactly the accepted rows: acc_h (host) gives the
        packed row count; the rows are built on the device from the sampler's outputs."""
        B = acc.shape[0]
        counts = acc.to(torch.int64) + 1
        total = sum(acc_h) + B
        seq_of = torch.repeat_interleave(torch.arange(B, device="cuda"), counts, output_size=total)
        cu = torch.zeros(B + 1, dtype=torch.int64, device="cuda")
        torch.cumsum(counts, 0, out=cu[1:])
        j = torch.arange(total, device="cuda") - cu[seq_of]
        tree_rows = seq_of * T + path.to(torch.int64)[seq_of, j]
        ids = out_tokens.to(torch.int64)[seq_of, j]
        pos = ctx_d[seq_of] + j
        slots = self._slots_of(block_tables, seq_of, pos)
        max_after = max(c + a + 1 for c, a in zip(ctx, acc_h))
        set_context(True, cu.to(torch.int32), None, max(acc_h) + 1, max_after, slots,
                    (ctx_d + counts).to(torch.int32), block_tables)
        feats_in = self.draft.fuse(aux[tree_rows])
        normed, feats = self.draft(ids, pos, feats_in)
        reset_context()
        return self._draft_state(normed, feats, cu[1:] - 1)
