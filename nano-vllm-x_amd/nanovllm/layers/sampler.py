"""Sampler and speculative rejection sampler on libnvx_spec (gfx950 HIP kernels).

* ``temperature_softmax`` -- fp32 ``softmax(logits.float() / T)`` per row, the first
  two lines of the reference's ``Sampler.forward`` (nanovllm/layers/sampler.py:9-10).
  Rows with temperature 0 are greedy and keep their fp32 logits.
* ``Sampler()(logits, temperatures)`` -- drop-in for sampler.py:5-12: one categorical
  draw per row (an inverse-CDF draw with device uniforms instead of the reference's
  exponential race; same distribution).  Greedy rows (temperature 0) take the argmax,
  which the reference forbids at sampling_params.py:11.
* ``rejection_sample_tree`` / ``rejection_sample_chain`` / ``RejectionSampler`` --
  speculative verification of a draft tree / chain (absent in the reference).
* ``topk_logprobs`` -- the k most likely tokens of ``log_softmax(logits)`` per row in
  one pass (the draft head's tree expansion; absent in the reference).
"""
import torch
from torch import nn

from .. import _C

_DTYPE_CODE = {torch.float32: _C.DTYPE_F32, torch.bfloat16: _C.DTYPE_BF16}


def temperature_softmax(logits: torch.Tensor, temperatures: torch.Tensor, out=None):
    """logits [N, V] (fp32 or bf16, unit stride in V); temperatures fp32 [N]."""
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("temperature_softmax: logits must be [N, V] with unit stride in V")
    if logits.dtype not in _DTYPE_CODE:
        raise ValueError(f"temperature_softmax: unsupported logits dtype {logits.dtype}")
    N, V = logits.shape
    temperatures = temperatures.to(device=logits.device, dtype=torch.float32).contiguous()
    if temperatures.numel() != N:
        raise ValueError("temperature_softmax: one temperature per row")
    probs = torch.empty(N, V, dtype=torch.float32, device=logits.device) if out is None else out
    _C.require_cuda(logits, temperatures, probs)
    _C.check(_C.lib().nvx_temperature_softmax(
        _C.ptr(logits), _DTYPE_CODE[logits.dtype], logits.stride(0), _C.ptr(temperatures),
        _C.ptr(probs), N, V, _C.stream_of(logits)))
    return probs


def topk_logprobs(logits: torch.Tensor, k: int):
    """Top-k of ``log_softmax(logits.float())`` per row: returns (log-probs fp32
    [N, k], tokens int64 [N, k]) in the order of ``torch.topk`` (descending; equal
    values by the lower token id).  logits [N, V] bf16 or fp32 with unit stride in V,
    16-byte aligned rows."""
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("topk_logprobs: logits must be [N, V] with unit stride in V")
    if logits.dtype not in _DTYPE_CODE:
        raise ValueError(f"topk_logprobs: unsupported logits dtype {logits.dtype}")
    N, V = logits.shape
    tok = torch.empty(N, k, dtype=torch.int32, device=logits.device)
    lp = torch.empty(N, k, dtype=torch.float32, device=logits.device)
    _C.require_cuda(logits)
    _C.check(_C.lib().nvx_topk_logprobs(
        _C.ptr(logits), _DTYPE_CODE[logits.dtype], logits.stride(0), N, V, k, _C.ptr(tok),
        _C.ptr(lp), _C.stream_of(logits)))
    return lp, tok.long()


def _i32(t):
    return t.to(torch.int32).contiguous()


_WALK_WS = {}  # (device index, stream) -> zero-filled uint8 tensor, grown on demand


def walk_workspace(num_seqs, device, workspace=None):
    """(tensor, bytes) of the exchange workspace for a walk of num_seqs sequences on the
    current stream of `device`.  The walk spreads each sequence over several
    workgroups, which meet through this memory; it must be zero-filled before its first
    use and is then owned by the library (it keeps per-sequence exchange counters).
    One workspace per (device, stream): walks on one stream run in order, and walks on
    different streams never share one.  A workspace passed in is used as given (the
    caller zero-fills it once and keeps it for walks that never overlap).  Under stream
    capture the walk runs one workgroup per sequence and takes none."""
    if workspace is not None:
        return workspace, workspace.numel() * workspace.element_size()
    if torch.cuda.is_current_stream_capturing():
        return None, 0
    need = _C.lib().nvx_rejection_walk_workspace_size(num_seqs)
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    ws = _WALK_WS.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(max(need, _C.lib().nvx_rejection_walk_workspace_size(256)),
                         dtype=torch.uint8, device=device)
        _WALK_WS[key] = ws
    return ws, ws.numel()


def rejection_sample_tree(target_probs, draft_probs, tokens, parents, uniforms, final_uniforms,
                          greedy=None, num_nodes=None, draft_mode="stochastic", workspace=None):
    """Verify one draft tree per sequence.

    target_probs fp32 [B, T, V] (row i: target distribution after node i);
    draft_probs fp32 [B, T', V] (row i: distribution that proposed node i's children,
    T' >= number of internal-node rows used) or None with draft_mode="delta";
    tokens, parents int [B, T] (parents[:, 0] = -1, parents[b, i] < i);
    uniforms fp32 [B, T]; final_uniforms fp32 [B]; greedy bool [B] or None;
    num_nodes int [B] or None (ragged trees); workspace: the walk's exchange memory
    (see walk_workspace; by default one kept per device and stream).

    Returns int32 (path [B, T], accepted_len [B], out_tokens [B, T], next_token [B]).
    accepted_len is -1 for a sequence whose workgroups failed to meet (callers check).
    """
    B, T, V = target_probs.shape
    if target_probs.dtype != torch.float32 or target_probs.stride(2) != 1 \
            or target_probs.stride(1) != V:
        raise ValueError("rejection_sample_tree: target_probs must be fp32 with contiguous rows")
    delta = draft_mode == "delta"
    if not delta:
        if draft_probs is None or draft_probs.dtype != torch.float32 or \
                draft_probs.stride(2) != 1 or draft_probs.stride(1) != V or draft_probs.shape[2] != V:
            raise ValueError("rejection_sample_tree: draft_probs must be fp32 [B, T', V] with "
                             "contiguous rows")
    if T > 64:
        raise ValueError("rejection_sample_tree: at most 64 nodes per tree")
    dev = target_probs.device
    tokens, parents = _i32(tokens), _i32(parents)
    uniforms = uniforms.to(torch.float32).contiguous()
    final_uniforms = final_uniforms.to(torch.float32).contiguous()
    g = None if greedy is None else greedy.to(device=dev, dtype=torch.uint8).contiguous()
    nn_ = None if num_nodes is None else _i32(num_nodes)
    path = torch.empty(B, T, dtype=torch.int32, device=dev)
    acc = torch.empty(B, dtype=torch.int32, device=dev)
    out_tokens = torch.empty(B, T, dtype=torch.int32, device=dev)
    nxt = torch.empty(B, dtype=torch.int32, device=dev)
    _C.require_cuda(target_probs, draft_probs, tokens, parents, uniforms, final_uniforms, g, nn_,
                    workspace)
    ws, ws_bytes = walk_workspace(B, dev, workspace)
    _C.check(_C.lib().nvx_rejection_sample_tree(
        _C.ptr(target_probs), target_probs.stride(0), None if delta else _C.ptr(draft_probs),
        0 if delta else draft_probs.stride(0), V, _C.ptr(tokens), _C.ptr(parents), _C.ptr(nn_), T,
        _C.ptr(uniforms), _C.ptr(final_uniforms), _C.ptr(g), 1 if delta else 0, B, _C.ptr(path),
        _C.ptr(acc), _C.ptr(out_tokens), _C.ptr(nxt), _C.ptr(ws), ws_bytes,
        _C.stream_of(target_probs)))
    return path, acc, out_tokens, nxt


def stats_eligible(logits: torch.Tensor) -> bool:
    """Whether logits [N, V] can take the fused path (softmax_stats and
    rejection_sample_tree_logits): bf16 or fp32, unit stride in V, 16-byte aligned
    rows, V and the row stride multiples of 8 (bf16) or 4 (fp32)."""
    if logits.dim() != 2 or logits.stride(1) != 1 or logits.dtype not in _DTYPE_CODE:
        return False
    per = 8 if logits.dtype == torch.bfloat16 else 4
    return (logits.shape[1] % per == 0 and logits.stride(0) % per == 0
            and logits.data_ptr() % 16 == 0)


def softmax_stats(logits: torch.Tensor, temperatures: torch.Tensor):
    """Per-row softmax statistics in one streaming pass, without writing probabilities:
    fp32 [N, 2] = (max(logits) * log2(e) / T, 1 / sum exp2(logits * log2(e) / T - max)),
    within 1e-5 relative of the exact values; rows with T == 0 get (0, 0)."""
    if not stats_eligible(logits):
        raise ValueError("softmax_stats: logits must be bf16/fp32 [N, V] with 16-byte aligned rows "
                         "and V, row stride multiples of 8 (bf16) or 4 (fp32)")
    N, V = logits.shape
    temperatures = temperatures.to(device=logits.device, dtype=torch.float32).contiguous()
    if temperatures.numel() != N:
        raise ValueError("softmax_stats: one temperature per row")
    stats = torch.empty(N, 2, dtype=torch.float32, device=logits.device)
    _C.require_cuda(logits, temperatures, stats)
    _C.check(_C.lib().nvx_softmax_stats(_C.ptr(logits), _DTYPE_CODE[logits.dtype], logits.stride(0),
                                        _C.ptr(temperatures), _C.ptr(stats), N, V,
                                        _C.stream_of(logits)))
    return stats


def softmax_from_stats(logits: torch.Tensor, temperatures: torch.Tensor, stats: torch.Tensor):
    """fp32 [N, V] probabilities exp2(fma(x, log2(e)/T, -stats[:, 0])) * stats[:, 1] (x at
    T == 0): the values rejection_sample_tree_logits uses for the same statistics."""
    if not stats_eligible(logits):
        raise ValueError("softmax_from_stats: logits must be bf16/fp32 [N, V] with 16-byte aligned "
                         "rows and V, row stride multiples of 8 (bf16) or 4 (fp32)")
    N, V = logits.shape
    temperatures = temperatures.to(device=logits.device, dtype=torch.float32).contiguous()
    stats = stats.to(torch.float32).contiguous()
    if temperatures.numel() != N or stats.shape != (N, 2):
        raise ValueError("softmax_from_stats: one temperature and one stats row per logits row")
    probs = torch.empty(N, V, dtype=torch.float32, device=logits.device)
    _C.require_cuda(logits, temperatures, stats, probs)
    _C.check(_C.lib().nvx_softmax_from_stats(_C.ptr(logits), _DTYPE_CODE[logits.dtype],
                                             logits.stride(0), _C.ptr(temperatures), _C.ptr(stats),
                                             _C.ptr(probs), N, V, _C.stream_of(logits)))
    return probs


def rejection_sample_tree_logits(logits, temperatures, stats, draft_probs, tokens, parents,
                                 uniforms, final_uniforms, greedy=None, num_nodes=None,
                                 draft_mode="stochastic", workspace=None):
    """rejection_sample_tree with the target rows given as logits [B*T, V] (row b*T + i
    for node i of sequence b), their temperatures [B*T] and softmax_stats: each
    probability the walk reads is recomputed from the logits and statistics, so the
    results equal rejection_sample_tree(softmax_from_stats(logits, temperatures, stats))."""
    B, T = tokens.shape
    if not stats_eligible(logits) or logits.shape[0] != B * T:
        raise ValueError("rejection_sample_tree_logits: logits must be [B*T, V] (see stats_eligible)")
    V = logits.shape[1]
    delta = draft_mode == "delta"
    if not delta:
        if draft_probs is None or draft_probs.dtype != torch.float32 or \
                draft_probs.stride(2) != 1 or draft_probs.stride(1) != V or draft_probs.shape[2] != V:
            raise ValueError("rejection_sample_tree_logits: draft_probs must be fp32 [B, T', V] "
                             "with contiguous rows")
    if T > 64:
        raise ValueError("rejection_sample_tree_logits: at most 64 nodes per tree")
    dev = logits.device
    temperatures = temperatures.to(device=dev, dtype=torch.float32).contiguous()
    stats = stats.to(torch.float32).contiguous()
    if temperatures.numel() != B * T or stats.shape != (B * T, 2):
        raise ValueError("rejection_sample_tree_logits: one temperature and one stats row per logits row")
    tokens, parents = _i32(tokens), _i32(parents)
    uniforms = uniforms.to(torch.float32).contiguous()
    final_uniforms = final_uniforms.to(torch.float32).contiguous()
    g = None if greedy is None else greedy.to(device=dev, dtype=torch.uint8).contiguous()
    nn_ = None if num_nodes is None else _i32(num_nodes)
    path = torch.empty(B, T, dtype=torch.int32, device=dev)
    acc = torch.empty(B, dtype=torch.int32, device=dev)
    out_tokens = torch.empty(B, T, dtype=torch.int32, device=dev)
    nxt = torch.empty(B, dtype=torch.int32, device=dev)
    _C.require_cuda(logits, temperatures, stats, draft_probs, tokens, parents, uniforms,
                    final_uniforms, g, nn_, workspace)
    ws, ws_bytes = walk_workspace(B, dev, workspace)
    _C.check(_C.lib().nvx_rejection_sample_tree_logits(
        _C.ptr(logits), _DTYPE_CODE[logits.dtype], logits.stride(0), _C.ptr(temperatures),
        _C.ptr(stats), None if delta else _C.ptr(draft_probs), 0 if delta else draft_probs.stride(0),
        V, _C.ptr(tokens), _C.ptr(parents), _C.ptr(nn_), T, _C.ptr(uniforms), _C.ptr(final_uniforms),
        _C.ptr(g), 1 if delta else 0, B, _C.ptr(path), _C.ptr(acc), _C.ptr(out_tokens), _C.ptr(nxt),
        _C.ptr(ws), ws_bytes, _C.stream_of(logits)))
    return path, acc, out_tokens, nxt


def rejection_sample_tree_logits_lazy(logits, temperatures, draft_probs, tokens, parents, uniforms,
                                      final_uniforms, greedy=None, num_nodes=None,
                                      draft_mode="stochastic", workspace=None, stats_out=None):
    """rejection_sample_tree on logits [B*T, V] (row b*T + i for node i of sequence b) and
    their temperatures [B*T], with no separate statistics pass: the walk computes the
    softmax statistics of the rows it visits (exact row max, then the sum in its
    canonical order) and writes them to stats_out (fp32 [B*T, 2], when given; rows the
    walk does not visit are left as they were).  The results equal
    rejection_sample_tree(softmax_from_stats(logits, temperatures, stats)) for any stats
    that hold stats_out's values on the visited rows.  Returns (path, accepted_len,
    out_tokens, next_token, stats_out)."""
    B, T = tokens.shape
    if not stats_eligible(logits) or logits.shape[0] != B * T:
        raise ValueError("rejection_sample_tree_logits_lazy: logits must be [B*T, V] "
                         "(see stats_eligible)")
    V = logits.shape[1]
    delta = draft_mode == "delta"
    if not delta:
        if draft_probs is None or draft_probs.dtype != torch.float32 or \
                draft_probs.stride(2) != 1 or draft_probs.stride(1) != V or draft_probs.shape[2] != V:
            raise ValueError("rejection_sample_tree_logits_lazy: draft_probs must be fp32 "
                             "[B, T', V] with contiguous rows")
    if T > 64:
        raise ValueError("rejection_sample_tree_logits_lazy: at most 64 nodes per tree")
    dev = logits.device
    temperatures = temperatures.to(device=dev, dtype=torch.float32).contiguous()
    if temperatures.numel() != B * T:
        raise ValueError("rejection_sample_tree_logits_lazy: one temperature per logits row")
    if stats_out is not None and (stats_out.shape != (B * T, 2) or stats_out.dtype != torch.float32
                                  or not stats_out.is_contiguous()):
        raise ValueError("rejection_sample_tree_logits_lazy: stats_out must be contiguous fp32 "
                         "[B*T, 2]")
    tokens, parents = _i32(tokens), _i32(parents)
    uniforms = uniforms.to(torch.float32).contiguous()
    final_uniforms = final_uniforms.to(torch.float32).contiguous()
    g = None if greedy is None else greedy.to(device=dev, dtype=torch.uint8).contiguous()
    nn_ = None if num_nodes is None else _i32(num_nodes)
    path = torch.empty(B, T, dtype=torch.int32, device=dev)
    acc = torch.empty(B, dtype=torch.int32, device=dev)
    out_tokens = torch.empty(B, T, dtype=torch.int32, device=dev)
    nxt = torch.empty(B, dtype=torch.int32, device=dev)
    _C.require_cuda(logits, temperatures, draft_probs, tokens, parents, uniforms, final_uniforms,
                    g, nn_, workspace, stats_out)
    ws, ws_bytes = walk_workspace(B, dev, workspace)
    _C.check(_C.lib().nvx_rejection_sample_tree_logits_lazy(
        _C.ptr(logits), _DTYPE_CODE[logits.dtype], logits.stride(0), _C.ptr(temperatures),
        _C.ptr(stats_out), None if delta else _C.ptr(draft_probs),
        0 if delta else draft_probs.stride(0), V, _C.ptr(tokens), _C.ptr(parents), _C.ptr(nn_), T,
        _C.ptr(uniforms), _C.ptr(final_uniforms), _C.ptr(g), 1 if delta else 0, B, _C.ptr(path),
        _C.ptr(acc), _C.ptr(out_tokens), _C.ptr(nxt), _C.ptr(ws), ws_bytes, _C.stream_of(logits)))
    return path, acc, out_tokens, nxt, stats_out


def rejection_sample_chain(target_probs, draft_probs, draft_token_ids, uniforms, final_uniforms,
                           greedy=None):
    """Chain speculative sampling (Leviathan et al. 2023, Alg. 1).

    target_probs fp32 [B, k+1, V]; draft_probs fp32 [B, k, V]; draft_token_ids [B, k];
    uniforms [B, k]; final_uniforms [B].  Returns int32 (accepted_len [B],
    recovered [B] (-1 when every draft token was accepted), bonus [B] (-1 otherwise),
    tokens [B, k+1] (accepted tokens then the recovered/bonus token, -1 padded)).
    """
    B, k1, V = target_probs.shape
    k = k1 - 1
    dev = target_probs.device
    tok = torch.zeros(B, k1, dtype=torch.int32, device=dev)
    tok[:, 1:] = draft_token_ids.to(torch.int32)
    u = torch.zeros(B, k1, dtype=torch.float32, device=dev)
    u[:, 1:] = uniforms
    parents = (torch.arange(k1, dtype=torch.int32, device=dev) - 1).expand(B, k1).contiguous()
    _, acc, toks, nxt = rejection_sample_tree(target_probs, draft_probs, tok, parents, u,
                                              final_uniforms, greedy)
    full = acc == k
    recovered = torch.where(full, torch.full_like(nxt, -1), nxt)
    bonus = torch.where(full, nxt, torch.full_like(nxt, -1))
    return acc, recovered, bonus, toks


class Sampler(nn.Module):
    """Sampler()(logits [N, V], temperatures [N]) -> int64 token ids [N]."""

    def forward(self, logits: torch.Tensor, temperatures: torch.Tensor, uniforms=None):
        N, V = logits.shape
        probs = temperature_softmax(logits, temperatures)
        dev = logits.device
        u = torch.rand(N, device=dev) if uniforms is None else uniforms
        zeros = torch.zeros(N, 1, dtype=torch.int32, device=dev)
        greedy = temperatures.to(dev) == 0
        _, _, _, nxt = rejection_sample_tree(probs.view(N, 1, V), None, zeros, zeros - 1,
                                             zeros.float(), u, greedy, draft_mode="delta")
        return nxt.long()


class RejectionSampler(nn.Module):
    """Temperature softmax of the target logits followed by tree verification.  When the
    logits qualify (stats_eligible) the softmax is fused into the walk: the walk
    computes the statistics of the rows it visits and recomputes each probability it
    reads (rejection_sample_tree_logits_lazy; lazy=False instead runs one statistics
    pass over every row first, softmax_stats + rejection_sample_tree_logits).
    Otherwise temperature_softmax then rejection_sample_tree.

    forward(target_logits [B*T, V], temperatures [B], draft_probs [B, T, V] | None,
    tokens [B, T], parents [B, T], uniforms [B, T], final_uniforms [B], num_nodes=None,
    stats_out=None) -> (path, accepted_len, out_tokens, next_token), int32.  stats_out
    (fp32 [B*T, 2]) receives the statistics of the visited rows on the lazy path.
    """

    def __init__(self, lazy=True):
        super().__init__()
        self.lazy = lazy

    def forward(self, target_logits, temperatures, draft_probs, tokens, parents, uniforms,
                final_uniforms, num_nodes=None, stats_out=None):
        B, T = tokens.shape
        V = target_logits.shape[-1]
        temps = temperatures.to(device=target_logits.device, dtype=torch.float32)
        rows = target_logits.view(B * T, V)
        row_temps = temps.repeat_interleave(T)
        mode = "delta" if draft_probs is None else "stochastic"
        if stats_eligible(rows) and self.lazy:
            return rejection_sample_tree_logits_lazy(rows, row_temps, draft_probs, tokens, parents,
                                                     uniforms, final_uniforms, temps == 0,
                                                     num_nodes, mode, stats_out=stats_out)[:4]
        if stats_eligible(rows):
            # fused: one statistics pass over the logits, then the walk recomputes the
            # probabilities of the rows it visits (no fp32 probability rows written)
            stats = softmax_stats(rows, row_temps)
            return rejection_sample_tree_logits(rows, row_temps, stats, draft_probs, tokens, parents,
                                                uniforms, final_uniforms, temps == 0, num_nodes, mode)
        probs = temperature_softmax(rows, row_temps)
        return rejection_sample_tree(probs.view(B, T, V), draft_probs, tokens, parents, uniforms,
                                     final_uniforms, temps == 0, num_nodes, mode)
