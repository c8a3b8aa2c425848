"""Fused last-position token sampler on the HIP kernel (csrc/sample.hip).

`sample_tokens(logits, temperature, seed, offset)` replaces the reference's batched sampling
(chat.py:103-107: softmax(logits.float() / temperature), torch.multinomial(probs, 1)) with one pass
over the logits: token = argmax_v(logit_v / T - ln E_v), E_v ~ Exp(1), the exponential race that
torch.multinomial itself uses for one sample, so the draws follow softmax(logits / T).  The random
numbers come from Philox4x32-10 keyed by `seed` at counter (v / 4, row, offset): callers advance
`offset` once per call.  temperature <= 0 is greedy.  A row with no candidate gets -1.
No CPU path: CPU tensors are rejected.
"""
import torch

from . import _lib

DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

_WORKSPACES = {}
_RETIRED = []   # outgrown buffers: never freed (a captured graph may still use one)


def _workspace(nbytes, device):
    """The sampler's partials buffer of (device, current stream), grown on demand, uninitialised
    (every slot the reduction reads is written by the same call); an outgrown buffer is kept
    alive, as a graph that captured a call holds its address."""
    if not nbytes:
        return None
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        size = int(nbytes)
        if ws is not None:
            _RETIRED.append(ws)
            # at least double: a workspace that grows step by step (one split more every 128
            # keys of a growing row) retires O(log) buffers whose sizes sum to less than its own
            size = max(size, 2 * ws.numel())
        ws = torch.empty(size, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def sample_tokens(logits, temperature, seed, offset, out=None):
    """logits [batch, vocab] (bf16, fp16 or fp32; rows may be strided) -> int32 tokens [batch]."""
    assert logits.is_cuda, "sample_tokens runs on the GPU only"
    assert logits.dim() == 2 and logits.stride(1) == 1, "logits must be [batch, vocab], unit stride"
    assert logits.dtype in DTYPES, f"logits must be bf16, fp16 or fp32, got {logits.dtype}"
    B, V = logits.shape
    if out is None:
        out = torch.empty(B, dtype=torch.int32, device=logits.device)
    assert out.dtype == torch.int32 and out.shape == (B,) and out.is_contiguous()
    lib = _lib.load()
    nbytes = lib.mi_fa2_sample_workspace_size(B, V)
    ws = _workspace(nbytes, logits.device)
    with torch.cuda.device(logits.device):
        _lib.check(lib.mi_fa2_sample(
            DTYPES[logits.dtype], logits.data_ptr(), logits.stride(0) if B > 1 else V, B, V,
            float(temperature), int(seed) & (2**64 - 1), int(offset) & (2**64 - 1),
            out.data_ptr(), ws.data_ptr() if ws is not None else None,
            ws.numel() if ws is not None else 0, _lib.stream_of(logits)))
    return out
