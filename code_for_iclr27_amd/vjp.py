"""The audit's margin objective and its gradients on the HIP path: drop-ins for
``last_token_logits_float32``, ``one_vs_rest_margin`` and ``one_vs_rest_hidden_gradient``
(src/lazy_recall/_core/scoring.py:27-76), ``row_margins`` and ``row_hidden_gradients``
(batch_audit.py:11-24), and the per-layer pre-projection gradient that ``compute_score_table``
forms from each layer's attention-output gradient (scoring.py:228-237).

Same names, arguments, shapes and f32 results as the reference. The reference runs these as
chunked torch GEMMs over f32 copies of the weight; here each is one pass of a HIP kernel
(liblazyrecall_hip.so: lr_head_logits, lr_margin_stats, lr_hidden_gradient, lr_pre_gradient)
over the weight in its stored dtype. ``chunk_size`` is accepted for signature parity and does
not change the result's definition. There is no CPU path.
"""

from __future__ import annotations

import torch

from . import _lib

_WEIGHT_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _check(condition: bool, message: str) -> None:
    if not condition:
        raise RuntimeError(message)


def _weight(tensor: torch.Tensor) -> torch.Tensor:
    _check(tensor.is_cuda, "Expected contiguous CUDA tensor")
    _check(tensor.dtype in _WEIGHT_DTYPES, "Weights must be float32, float16 or bfloat16")
    return tensor.detach().contiguous()


def _output_embeddings(model):
    output = model.get_output_embeddings()
    if output is None or not hasattr(output, "weight"):
        raise RuntimeError("Model has no linear output embedding layer")
    return output


def _workspace(rows: int, vocab: int, dim: int, device) -> torch.Tensor:
    size = _lib.load().lr_row_sum_workspace_bytes(rows, vocab, dim)
    return torch.empty(max(size, 16), dtype=torch.uint8, device=device)


def _stats(logits: torch.Tensor, targets: torch.Tensor | None):
    rows, vocab = logits.shape
    device = logits.device
    margins = torch.empty(rows, dtype=torch.float32, device=device)
    stats = torch.empty((rows, 2), dtype=torch.float32, device=device)
    chosen = torch.empty(rows, dtype=torch.int64, device=device)
    size = _lib.load().lr_margin_stats_workspace_bytes(rows, vocab)
    workspace = torch.empty(max(size, 16), dtype=torch.uint8, device=device)
    _lib.call("lr_margin_stats", logits.data_ptr(), rows, vocab, _lib.ptr(targets),
              chosen.data_ptr(), margins.data_ptr(), stats.data_ptr(), workspace.data_ptr(),
              workspace.numel(), _lib.stream_of(logits))
    return margins, chosen, stats


def _logits_rows(logits: torch.Tensor) -> torch.Tensor:
    _check(logits.is_cuda, "Expected contiguous CUDA tensor")
    logits = logits.detach().float()
    return logits.reshape(-1, logits.shape[-1]).contiguous()


def last_token_logits_float32(model, final_hidden_state: torch.Tensor, chunk_size: int = 4096):
    """_core/scoring.py:34-52: f32 logits of the output head, [..., vocab]."""
    del chunk_size
    output = _output_embeddings(model)
    weight = _weight(output.weight)
    bias = getattr(output, "bias", None)
    bias = None if bias is None else bias.detach().to(weight.dtype).contiguous()
    hidden = final_hidden_state.detach().float()
    _check(hidden.is_cuda and hidden.device == weight.device, "CUDA devices differ")
    vocab, dim = weight.shape
    _check(hidden.shape[-1] == dim, "Hidden size differs from the output embedding")
    flat = hidden.reshape(-1, dim).contiguous()
    with torch.cuda.device(weight.device):
        out = torch.empty((flat.shape[0], vocab), dtype=torch.float32, device=weight.device)
        if flat.shape[0]:
            _lib.call("lr_head_logits", flat.data_ptr(), flat.shape[0], weight.data_ptr(),
                      _lib.ptr(bias), vocab, dim, _lib.DTYPE_CODES[weight.dtype], out.data_ptr(),
                      _lib.stream_of(weight))
    return out.reshape(*hidden.shape[:-1], vocab)


def one_vs_rest_margin(logits: torch.Tensor, target_id: int) -> torch.Tensor:
    """_core/scoring.py:27-31: logits[target] - logsumexp(all other logits), a 0-d f32 tensor."""
    flat = _logits_rows(logits).reshape(1, -1)
    target = torch.tensor([int(target_id)], dtype=torch.int64, device=flat.device)
    _check(0 <= int(target_id) < flat.shape[1], "index out of range")
    with torch.cuda.device(flat.device):
        margins, _, _ = _stats(flat, target)
    return margins[0]


def one_vs_rest_hidden_gradient(model, logits: torch.Tensor, target_id: int,
                                chunk_size: int = 4096) -> torch.Tensor:
    """_core/scoring.py:55-76: W[target] - softmax(competitors) @ W per logits row, f32 [rows, D]."""
    del chunk_size
    weight = _weight(model.get_output_embeddings().weight)
    rows = _logits_rows(logits)
    count, vocab = rows.shape
    _check(vocab == weight.shape[0], "Logits width differs from the output embedding")
    _check(0 <= int(target_id) < vocab, "index out of range")
    with torch.cuda.device(weight.device):
        targets = torch.full((count,), int(target_id), dtype=torch.int64, device=weight.device)
        return _gradient(rows, targets, weight, None)


def _gradient(rows, targets, weight, due):
    count, vocab = rows.shape
    dim = weight.shape[1]
    _, _, stats = _stats(rows, targets)
    out = torch.empty((count, dim), dtype=torch.float32, device=weight.device)
    workspace = _workspace(count, vocab, dim, weight.device)
    _lib.call("lr_hidden_gradient", rows.data_ptr(), stats.data_ptr(), targets.data_ptr(), count,
              weight.data_ptr(), vocab, dim, _lib.DTYPE_CODES[weight.dtype], _lib.ptr(due),
              out.data_ptr(), workspace.data_ptr(), workspace.numel(), _lib.stream_of(weight))
    return out


def row_margins(logits: torch.Tensor):
    """batch_audit.py:11-15 -> (margins [rows], targets [rows] i64, competitors [rows, vocab])."""
    rows = _logits_rows(logits)
    with torch.cuda.device(rows.device):
        margins, targets, _ = _stats(rows, None)
        competitors = rows.scatter(1, targets[:, None], -torch.inf)
    return margins, targets, competitors


def row_hidden_gradients(model, logits, targets, competitors, due, chunk_size=4096):
    """batch_audit.py:18-24: (W[target_r] - softmax(competitors_r) @ W) * due[r], f32 [rows, D]."""
    del competitors, chunk_size  # the competitor softmax is formed from logits and targets
    weight = _weight(model.get_output_embeddings().weight)
    rows = _logits_rows(logits)
    _check(rows.shape[1] == weight.shape[0], "Logits width differs from the output embedding")
    with torch.cuda.device(weight.device):
        targets = targets.to(device=weight.device, dtype=torch.int64).contiguous()
        due = torch.tensor(due, device=weight.device, dtype=torch.float32).reshape(-1)
        _check(targets.numel() == rows.shape[0] and due.numel() == rows.shape[0],
               "One target and one due flag per row")
        return _gradient(rows, targets, weight, due)


def pre_gradient(post_gradient: torch.Tensor, o_proj_weight: torch.Tensor, num_query_heads: int,
                 head_dim: int, gate: torch.Tensor | None = None) -> torch.Tensor:
    """scoring.py:228-237: (post_gradient @ o_proj.weight.float()).view(Hq, d) [* gate], f32."""
    weight = _weight(o_proj_weight)
    hidden, width = weight.shape
    _check(width == num_query_heads * head_dim, "o_proj width differs from Hq * head_dim")
    post = post_gradient.detach().float().reshape(-1).contiguous()
    _check(post.numel() == hidden and post.is_cuda, "Post-projection gradient size differs")
    if gate is not None:
        gate = gate.detach().float().reshape(-1).contiguous()
        _check(gate.numel() == width, "Missing current Qwen3.5 attention output gate")
    with torch.cuda.device(weight.device):
        out = torch.empty(width, dtype=torch.float32, device=weight.device)
        workspace = _workspace(1, hidden, width, weight.device)
        _lib.call("lr_pre_gradient", post.data_ptr(), weight.data_ptr(), hidden, width,
                  _lib.DTYPE_CODES[weight.dtype], _lib.ptr(gate), out.data_ptr(),
                  workspace.data_ptr(), workspace.numel(), _lib.stream_of(weight))
    return out.view(num_query_heads, head_dim)


def pre_gradients(post_gradients, o_proj_weights, num_query_heads: int, head_dim: int,
                  gates=None) -> list:
    """The pre-projection gradient of every layer (the per-layer lines of scoring.py:228-237 over
    all layers) in one launch pair: a list of f32 [Hq, d] tensors, layer by layer."""
    layers = len(o_proj_weights)
    _check(layers > 0 and len(post_gradients) == layers, "One post gradient per layer")
    gates = [None] * layers if gates is None else list(gates)
    _check(len(gates) == layers, "One gate (or None) per layer")
    weights = [_weight(w) for w in o_proj_weights]
    hidden, width = weights[0].shape
    device, dtype = weights[0].device, weights[0].dtype
    _check(all(w.shape == (hidden, width) and w.dtype == dtype and w.device == device
               for w in weights), "Every o_proj must share shape, dtype and device")
    _check(width == num_query_heads * head_dim, "o_proj width differs from Hq * head_dim")
    # the kernels read weight rows 16 bytes at a time; the device table hides the addresses
    # from the library's own check, so it is made here
    _check(all(w.data_ptr() % 16 == 0 for w in weights), "Weights must be 16-byte aligned")
    posts = [p.detach().float().reshape(-1).contiguous() for p in post_gradients]
    _check(all(p.numel() == hidden and p.device == device for p in posts),
           "Post-projection gradient size differs")
    gates = [None if g is None else g.detach().float().reshape(-1).contiguous() for g in gates]
    _check(all(g is None or (g.numel() == width and g.device == device) for g in gates),
           "Missing current Qwen3.5 attention output gate")
    with torch.cuda.device(device):
        out = torch.empty((layers, width), dtype=torch.float32, device=device)
        table = torch.tensor([[w.data_ptr(), p.data_ptr(), 0 if g is None else g.data_ptr(),
                               out[l].data_ptr()]
                              for l, (w, p, g) in enumerate(zip(weights, posts, gates))],
                             dtype=torch.int64).pin_memory().to(device, non_blocking=True)
        size = _lib.load().lr_pre_gradient_layers_workspace_bytes(layers, hidden, width)
        workspace = torch.empty(max(size, 16), dtype=torch.uint8, device=device)
        _lib.call("lr_pre_gradient_layers", table.data_ptr(), layers, hidden, width,
                  _lib.DTYPE_CODES[dtype], workspace.data_ptr(), workspace.numel(),
                  _lib.stream_of(weights[0]))
        # the table and the inputs stay referenced until the launch pair has run
        out._lr_keepalive = (table, posts, gates, weights)
    return [out[l].view(num_query_heads, head_dim) for l in range(layers)]
