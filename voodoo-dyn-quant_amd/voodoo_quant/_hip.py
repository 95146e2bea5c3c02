"""ctypes binding of ``libvoodoo_hip.so`` (declared in ``include/voodoo_hip.h``).

Tensors cross the boundary as raw device pointers; every call is enqueued on
the caller's current HIP stream.  There is no fallback: if the library is not
built, or a tensor is not on a ROCm device, calls raise.
"""

from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path

import torch

_LIB_PATH = Path(os.environ.get("VOODOO_HIP_LIB", Path(__file__).resolve().parent / "libvoodoo_hip.so"))
_LIB = None

VQ_OK, VQ_ERR_QTYPE, VQ_ERR_ALIGN, VQ_ERR_NULL, VQ_ERR_SHAPE, VQ_ERR_HIP, VQ_ERR_WORKSPACE = range(7)

# (name, restype, argtypes) for every entry point of include/voodoo_hip.h
_i, _i64, _p = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
_SIGNATURES = [
    ("vq_version", _i, []),
    ("vq_last_error_string", ctypes.c_char_p, []),
    ("vq_group_bytes", _i64, [_i]),
    ("vq_qbytes_size", _i64, [_i, _i64, _i64]),
    ("vq_validate_candidates", _i, [_i, _p, _i64, _i64, _i64]),
    ("vq_dequant", _i, [_i, _p, _p, _i64, _i64, _p]),
    ("vq_dequant_bf16", _i, [_i, _p, _p, _i64, _i64, _p]),
    ("vq_mix_weight", _i, [_i, _p, _p, _p, _i64, _i64, _p, _p]),
    ("vq_routed_linear_fwd", _i, [_p, _i64, _i64, _i64, _i64, _i, _p, _p, _p, _p, _p]),
    ("vq_embedding_rows_fwd", _i, [_i, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _i, _p]),
    ("vq_embedding_rows_bwd_workspace", _i64, [_i64, _i64, _i]),
    ("vq_embedding_rows_bwd", _i, [_i, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _i, _p, _p, _i64, _p]),
    ("vq_linear_fwd", _i, [_p, _i64, _i64, _i64, _p, _i64, _p, _p, _i64, _p]),
    ("vq_gated_linear_group_fwd", _i, [_p, _i64, _i64, _i64, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p]),
    ("vq_gated_linear_group_bwd_workspace", _i64, [_i64, _i64, _i, _p, _p]),
    ("vq_gated_linear_group_bwd", _i, [_p, _p, _i64, _i64, _i64, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p]),
    ("vq_gated_linear_group_bwd_gate_stream", _i,
     [_p, _p, _i64, _i64, _i64, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p]),
    ("vq_rope_qkv_fwd", _i, [_p, _i64, _i64, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p]),
    ("vq_rope_qkv_bwd", _i, [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i, _i, _i, _p, _p, _p, _p]),
    ("vq_swiglu_fwd", _i, [_p, _i64, _i64, _p, _p]),
    ("vq_swiglu_bwd", _i, [_p, _p, _i64, _i64, _p, _p]),
    ("vq_add_rmsnorm_fwd", _i, [_p, _p, _p, _i64, _i64, ctypes.c_float, _p, _p, _p, _p]),
    ("vq_rmsnorm_bwd", _i, [_p, _p, _p, _p, _p, _i64, _i64, _p, _p]),
    ("vq_attention_fwd", _i, [_p, _p, _p, _p, _p, _i64, _i64, _i, _i, _i, _p, _p, _p, _p, ctypes.c_float, _p]),
    ("vq_attention_bwd_workspace", _i64, [_i64, _i64, _i]),
    ("vq_attention_bwd", _i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i, _i, _i, _p, ctypes.c_float, _p,
                              _i64, _p]),
    ("vq_distill_loss_workspace", _i64, [_i64]),
    ("vq_distill_loss_fwd", _i, [_p, _p, _p, _i64, _i64, ctypes.c_float, _p, _p, _i64, _p]),
    ("vq_distill_loss_bwd", _i, [_p, _p, _p, _i64, _i64, ctypes.c_float, _p, _p, _p, _i64, _p]),
    ("vq_gated_linear_fwd_workspace", _i64, [_i64, _i64, _i64]),
    ("vq_gated_linear_fwd", _i, [_p, _i64, _i64, _i64, _i64, _i, _p, _p, _p, _p, _p, _p, _i64, _p]),
    ("vq_gated_linear_bwd_workspace", _i64, [_i64, _i64, _i64, _i64, _i, _i]),
    ("vq_gated_linear_bwd", _i, [_p, _p, _i64, _i64, _i64, _i64, _i, _p, _p, _p, _p, _p, _p, _p, _i64, _p]),
    ("vq_gated_linear_bwd_gate_stream", _i,
     [_p, _p, _i64, _i64, _i64, _i64, _i, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p]),
    ("vq_gated_linear_bwd_static", _i, [_p, _p, _i64, _i64, _i64, _i64, _i, _p, _p, _p, _p, _p, _p]),
    ("vq_gated_linear_fused_workspace", _i64, [_i64, _i64, _i64, _i]),
    ("vq_gated_linear_fwd_fused", _i, [_p, _i64, _i64, _i64, _i64, _i, _p, _p, _p, _p, _p, _i64, _p]),
    ("vq_gated_linear_dx_fused", _i, [_p, _i64, _i64, _i64, _i64, _i, _p, _p, _p, _p, _p, _i64, _p]),
]
EXPORTED = [s[0] for s in _SIGNATURES]


class HipLibraryError(RuntimeError):
    pass


def library_path() -> Path:
    return _LIB_PATH


def lib():
    """Load the shared library (once).  Raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not _LIB_PATH.exists():
            raise HipLibraryError(
                f"{_LIB_PATH} not found: build it with `python voodoo-dyn-quant_amd/build.py` "
                "(or __graft_entry__.build()); the gated Linear has no non-HIP path"
            )
        L = ctypes.CDLL(str(_LIB_PATH))
        for name, res, args in _SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def _raise(rc: int, what: str) -> None:
    msg = lib().vq_last_error_string().decode(errors="replace")
    if rc in (VQ_ERR_QTYPE, VQ_ERR_ALIGN, VQ_ERR_NULL, VQ_ERR_SHAPE):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (code {rc})")


def _check(rc: int, what: str) -> None:
    if rc != VQ_OK:
        _raise(rc, what)


def _dev_ptr(t: torch.Tensor | None, name: str) -> int | None:
    if t is None:
        return None
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a ROCm device, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _int_array(vals):
    arr = (ctypes.c_int * len(vals))(*vals)
    return arr


def _ptr_array(tensors, name):
    return (ctypes.c_void_p * len(tensors))(*[_dev_ptr(t, f"{name}[{i}]") for i, t in enumerate(tensors)])


# ----------------------------------------------------------------------------- host-side queries
def group_bytes(ggml_type: int) -> int:
    return int(lib().vq_group_bytes(ggml_type))


def qbytes_size(ggml_type: int, nrows: int, ncols: int) -> int:
    n = int(lib().vq_qbytes_size(ggml_type, nrows, ncols))
    if n < 0:
        _raise(VQ_ERR_ALIGN, "vq_qbytes_size")
    return n


def validate_candidates(ggml_types: list[int], n: int, d: int, d_pad: int) -> None:
    _check(lib().vq_validate_candidates(len(ggml_types), _int_array(ggml_types), n, d, d_pad),
           "vq_validate_candidates")


# ----------------------------------------------------------------------------- device calls
def dequant(ggml_type: int, qbytes: torch.Tensor, nrows: int, ncols: int, out: torch.Tensor | None = None):
    """fp32 [nrows, ncols] decode of packed bytes, bit-exact to ggml."""
    if out is None:
        out = torch.empty(nrows, ncols, dtype=torch.float32, device=qbytes.device)
    _check(lib().vq_dequant(ggml_type, _dev_ptr(qbytes, "qbytes"), _dev_ptr(out, "out"), nrows, ncols,
                            _stream(qbytes.device)), "vq_dequant")
    return out


def dequant_bf16(ggml_type: int, qbytes: torch.Tensor, nrows: int, ncols: int, out: torch.Tensor | None = None):
    """bf16 [nrows, ncols] of ggml's values (torch's rounding)."""
    if out is None:
        out = torch.empty(nrows, ncols, dtype=torch.bfloat16, device=qbytes.device)
    _check(lib().vq_dequant_bf16(ggml_type, _dev_ptr(qbytes, "qbytes"), _dev_ptr(out, "out"), nrows, ncols,
                                 _stream(qbytes.device)), "vq_dequant_bf16")
    return out


def routed_linear_fwd(x: torch.Tensor, cand_bf16, perm: torch.Tensor, group_off: torch.Tensor, n: int, d_pad: int,
                      y: torch.Tensor) -> None:
    """PTQR forward: y[perm[r]] = x[perm[r]] . cand_bf16[g]^T for the rows r of group g."""
    m, d = x.shape
    if perm.dtype != torch.int32 or group_off.dtype != torch.int32:
        raise ValueError("perm and group_off must be int32")
    _check(lib().vq_routed_linear_fwd(_dev_ptr(x, "x"), m, n, d, d_pad, len(cand_bf16),
                                      _ptr_array(cand_bf16, "cand_bf16"), _dev_ptr(perm, "perm"),
                                      _dev_ptr(group_off, "group_off"), _dev_ptr(y, "y"), _stream(x.device)),
           "vq_routed_linear_fwd")


def _ids(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.int64:
        raise ValueError(f"{name} must be int64, got {t.dtype}")
    return t


def embedding_rows_fwd(ggml_types, qbytes, probs: torch.Tensor | None, routing: torch.Tensor | None,
                       ids: torch.Tensor, num_embeddings: int, dim: int, d_pad: int,
                       dtype: torch.dtype = torch.bfloat16, out: torch.Tensor | None = None) -> torch.Tensor:
    """[len(ids), dim] in `dtype` (bf16 or fp32): rows `ids` of the mixture
    (routing None) or, per row r, of candidate routing[r] (PTQR)."""
    ids = _ids(ids, "ids")
    if routing is not None:
        routing = _ids(routing, "routing")
        if routing.numel() != ids.numel():
            raise ValueError(f"routing has {routing.numel()} entries for {ids.numel()} ids")
    if dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"embedding rows come as bf16 or fp32, not {dtype}")
    dev = ids.device
    if out is None:
        out = torch.empty(ids.numel(), dim, dtype=dtype, device=dev)
    elif out.dtype != dtype:
        raise ValueError(f"out is {out.dtype}, expected {dtype}")
    _check(lib().vq_embedding_rows_fwd(len(ggml_types), _int_array(ggml_types), _ptr_array(qbytes, "qbytes"),
                                       _dev_ptr(probs, "probs"), _dev_ptr(routing, "routing"), _dev_ptr(ids, "ids"),
                                       ids.numel(), num_embeddings, dim, d_pad, _dev_ptr(out, "out"),
                                       int(dtype == torch.float32), _stream(dev)),
           "vq_embedding_rows_fwd")
    return out


def embedding_rows_bwd(ggml_types, qbytes, ids: torch.Tensor, num_embeddings: int, dim: int, d_pad: int,
                       grad: torch.Tensor, dprobs: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 [K]: dprobs[k] = sum_r <grad[r], W_k[ids[r]][:dim]> (grad bf16 or fp32)."""
    ids = _ids(ids, "ids")
    dev = ids.device
    k = len(ggml_types)
    if grad.dtype not in (torch.bfloat16, torch.float32) or tuple(grad.shape) != (ids.numel(), dim):
        raise ValueError(f"grad must be bf16 or fp32 [{ids.numel()}, {dim}], got {grad.dtype} {tuple(grad.shape)}")
    if dprobs is None:
        dprobs = torch.empty(k, dtype=torch.float32, device=dev)
    nbytes = int(lib().vq_embedding_rows_bwd_workspace(ids.numel(), dim, k))
    if nbytes < 0:
        raise ValueError(f"invalid embedding sizes nids={ids.numel()} dim={dim} ncand={k}")
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    _check(lib().vq_embedding_rows_bwd(k, _int_array(ggml_types), _ptr_array(qbytes, "qbytes"), _dev_ptr(ids, "ids"),
                                       ids.numel(), num_embeddings, dim, d_pad, _dev_ptr(grad, "grad"),
                                       int(grad.dtype == torch.float32), _dev_ptr(dprobs, "dprobs"), _dev_ptr(ws, "workspace"), ws.numel(),
                                       _stream(dev)),
           "vq_embedding_rows_bwd")
    return dprobs


def mix_weight(ggml_types, qbytes, probs: torch.Tensor, n: int, d_pad: int, out: torch.Tensor | None = None):
    """bf16 [n, d_pad] W_eff = sum_k probs[k] * W_k (fp32, k-ordered)."""
    dev = probs.device
    if out is None:
        out = torch.empty(n, d_pad, dtype=torch.bfloat16, device=dev)
    _check(lib().vq_mix_weight(len(ggml_types), _int_array(ggml_types), _ptr_array(qbytes, "qbytes"),
                               _dev_ptr(probs, "probs"), n, d_pad, _dev_ptr(out, "w_eff"), _stream(dev)),
           "vq_mix_weight")
    return out


def fwd_workspace_bytes(m: int, n: int, d: int) -> int:
    v = int(lib().vq_gated_linear_fwd_workspace(m, n, d))
    if v < 0:
        raise ValueError(f"invalid forward sizes m={m} n={n} d={d}")
    return v


def linear_fwd(x: torch.Tensor, w: torch.Tensor, n: int, y: torch.Tensor,
               workspace: torch.Tensor | None = None) -> None:
    """y[m, :n] = x @ w[:n, :d]^T for a bf16 w with row stride w.shape[1]."""
    m, d = x.shape
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check(lib().vq_linear_fwd(_dev_ptr(x, "x"), m, n, d, _dev_ptr(w, "w"), w.shape[1], _dev_ptr(y, "y"),
                               _dev_ptr(workspace, "workspace"), ws_bytes, _stream(x.device)),
           "vq_linear_fwd")


def _group_arrays(members):
    """members: [(ggml_types, qbytes, n)] -> ctypes arrays (n, ncand, qtypes, qbytes)."""
    ns = (ctypes.c_int64 * len(members))(*[int(mb[2]) for mb in members])
    nc = (ctypes.c_int * len(members))(*[len(mb[0]) for mb in members])
    types = [t for mb in members for t in mb[0]]
    qbs = [q for mb in members for q in mb[1]]
    return ns, nc, _int_array(types), _ptr_array(qbs, "qbytes")


def gated_linear_group_fwd(x: torch.Tensor, members, probs, d_pad: int, w_eff: torch.Tensor, y: torch.Tensor,
                           workspace: torch.Tensor | None = None) -> None:
    """members: [(ggml_types, qbytes, n)]; probs: fp32 [K_i] per member.
    Writes w_eff [sum n, d_pad] and y [m, sum n]."""
    m, d = x.shape
    ns, nc, types, qbs = _group_arrays(members)
    pp = (ctypes.c_void_p * len(members))(*[_dev_ptr(p, f"probs[{i}]") for i, p in enumerate(probs)])
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check(lib().vq_gated_linear_group_fwd(_dev_ptr(x, "x"), m, d, d_pad, len(members), ns, nc, types, qbs, pp,
                                           _dev_ptr(w_eff, "w_eff"), _dev_ptr(y, "y"), _dev_ptr(workspace, "workspace"),
                                           ws_bytes, _stream(x.device)),
           "vq_gated_linear_group_fwd")


def group_bwd_workspace_bytes(m: int, d: int, members) -> int:
    ns, nc, _, _ = _group_arrays([(mb[0], [], mb[2]) for mb in members])
    v = int(lib().vq_gated_linear_group_bwd_workspace(m, d, len(members), ns, nc))
    if v < 0:
        raise ValueError(f"invalid group backward sizes m={m} d={d}")
    return v


def gated_linear_group_bwd(dy: torch.Tensor, x: torch.Tensor, members, d_pad: int, w_eff: torch.Tensor | None,
                           dx: torch.Tensor | None, dprobs: list | None, workspace: torch.Tensor | None,
                           gate_stream: torch.cuda.Stream | None = None) -> None:
    """gate_stream: finish the gate gradients (dot pass, reduce into dprobs)
    on that stream, after a fence on the current one."""
    m, d = x.shape
    ns, nc, types, qbs = _group_arrays(members)
    dp = None
    if dprobs is not None:
        dp = (ctypes.c_void_p * len(members))(*[_dev_ptr(t, f"dprobs[{i}]") for i, t in enumerate(dprobs)])
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    args = (_dev_ptr(dy, "dy"), _dev_ptr(x, "x"), m, d, d_pad, len(members), ns, nc, types, qbs,
            _dev_ptr(w_eff, "w_eff"), _dev_ptr(dx, "dx"), dp, _dev_ptr(workspace, "workspace"), ws_bytes,
            _stream(dy.device))
    if gate_stream is None:
        _check(lib().vq_gated_linear_group_bwd(*args), "vq_gated_linear_group_bwd")
    else:
        _check(lib().vq_gated_linear_group_bwd_gate_stream(*args, gate_stream.cuda_stream),
               "vq_gated_linear_group_bwd_gate_stream")


def mix_only_call(members, probs, d_pad: int, w_eff: torch.Tensor, stream: int):
    """A zero-argument callable that mixes `members` ([(ggml_types, qbytes, n)],
    stacked in order) with `probs` (one fp32 [K_i] tensor per member) into
    w_eff [sum n, d_pad] on `stream`: the tensors' addresses are marshalled
    once, so every call is one C call.  The tensors must outlive the callable
    and keep their storage."""
    if len(members) == 1:
        types, qbytes, n = members[0]
        args = (None, 0, n, d_pad, d_pad, len(types), _int_array(types), _ptr_array(qbytes, "qbytes"),
                _dev_ptr(probs[0], "probs"), _dev_ptr(w_eff, "w_eff"), None, None, 0, stream)
        fn, what = lib().vq_gated_linear_fwd, "vq_gated_linear_fwd"
    else:
        ns, nc, types, qbs = _group_arrays(members)
        pp = (ctypes.c_void_p * len(members))(*[_dev_ptr(p, f"probs[{i}]") for i, p in enumerate(probs)])
        args = (None, 0, d_pad, d_pad, len(members), ns, nc, types, qbs, pp, _dev_ptr(w_eff, "w_eff"), None, None, 0,
                stream)
        fn, what = lib().vq_gated_linear_group_fwd, "vq_gated_linear_group_fwd"

    def call() -> None:
        _check(fn(*args), what)

    call.keepalive = (args,)
    return call


def rope_qkv_fwd(qkv: torch.Tensor, B: int, S: int, Hq: int, Hkv: int, D: int, cos: torch.Tensor, sin: torch.Tensor,
                 repeat_kv: bool = True):
    """(q, k, v) from the stacked projection output: q bf16 [B*S, Hq, D],
    k and v [B*S, Hq, D] with each K/V head repeated (repeat_kv) or
    [B*S, Hkv, D]."""
    dev = qkv.device
    kv_out = Hq if repeat_kv else Hkv
    q = torch.empty(B * S, Hq, D, dtype=torch.bfloat16, device=dev)
    k, v = (torch.empty(B * S, kv_out, D, dtype=torch.bfloat16, device=dev) for _ in range(2))
    _check(lib().vq_rope_qkv_fwd(_dev_ptr(qkv, "qkv"), B, S, Hq, Hkv, kv_out, D, _dev_ptr(cos, "cos"),
                                 _dev_ptr(sin, "sin"), _dev_ptr(q, "q"), _dev_ptr(k, "k"), _dev_ptr(v, "v"),
                                 _stream(dev)),
           "vq_rope_qkv_fwd")
    return q, k, v


def rope_qkv_bwd(dq, dk, dv, B: int, S: int, Hq: int, Hkv: int, D: int, cos, sin) -> torch.Tensor:
    """dqkv bf16 [B*S, (Hq + 2 Hkv) D] from gradients shaped [B, Hq, S, D]
    (any strides with a unit stride along D; the three share them)."""
    dev = dq.device
    grads = [dq, dk, dv]
    if any(g.stride() != dq.stride() or g.stride(-1) != 1 for g in grads):
        grads = [g.contiguous() for g in grads]
    sb, sh, ss, _ = grads[0].stride()
    out = torch.empty(B * S, (Hq + 2 * Hkv) * D, dtype=torch.bfloat16, device=dev)
    ptr = [g.data_ptr() for g in grads]
    _check(lib().vq_rope_qkv_bwd(ptr[0], ptr[1], ptr[2], sb, sh, ss, B, S, Hq, Hkv, D, _dev_ptr(cos, "cos"),
                                 _dev_ptr(sin, "sin"), _dev_ptr(out, "dqkv"), _stream(dev)),
           "vq_rope_qkv_bwd")
    return out


def _bsh_strides(t: torch.Tensor, name: str):
    """(batch, position, head) element strides of a [B, H, S, D] bf16 tensor,
    copying it to the [B, S, H, D] layout when they do not suit the kernel."""
    if t.device.type != "cuda" or t.dtype != torch.bfloat16 or t.dim() != 4:
        raise ValueError(f"{name} must be a bf16 [B, H, S, D] tensor on a ROCm device")
    sb, sh, ss, sd = t.stride()
    if sd != 1 or sb % 8 or sh % 8 or ss % 8 or t.data_ptr() % 16:
        t = t.transpose(1, 2).contiguous().transpose(1, 2)
        sb, sh, ss, sd = t.stride()
    return t, (ctypes.c_int64 * 3)(sb, ss, sh)


def attention_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float | None = None,
                  need_lse: bool = True):
    """Causal attention forward, head dim 64: q [B, Hq, S, 64], k/v
    [B, Hk, S, 64] bf16 (Hq % Hk == 0) -> (out [B, Hq, S, 64] over
    [B, S, Hq, 64] memory, lse fp32 [B, Hq, S] natural log, or None)."""
    B, Hq, S, D = q.shape
    Hk = k.shape[1]
    if k.shape != (B, Hk, S, D) or v.shape != k.shape:
        raise ValueError(f"k/v shape {tuple(k.shape)}/{tuple(v.shape)} does not match q {tuple(q.shape)}")
    q, qs = _bsh_strides(q, "q")
    k, ks = _bsh_strides(k, "k")
    v, vs = _bsh_strides(v, "v")
    dev = q.device
    out = torch.empty(B, S, Hq, D, dtype=torch.bfloat16, device=dev).transpose(1, 2)
    os_ = (ctypes.c_int64 * 3)(out.stride(0), out.stride(2), out.stride(1))
    lse = torch.empty(B, Hq, S, dtype=torch.float32, device=dev) if need_lse else None
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(D)
    _check(lib().vq_attention_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                  lse.data_ptr() if lse is not None else None, B, S, Hq, Hk, D, qs, ks, vs, os_, sc,
                                  _stream(dev)),
           "vq_attention_fwd")
    return out, lse


def attention_bwd(dout: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                  lse: torch.Tensor, scale: float | None = None):
    """Backward of :func:`attention_fwd`: (dq, dk, dv), each bf16 [B, Hq, S, 64]
    over [B, S, Hq, 64] memory.  k and v may have Hk heads (Hq % Hk == 0):
    dk and dv are per query head either way, the gradients of K and V with
    each head repeated Hq/Hk times (K/V head j's gradient is the sum over
    query heads j*Hq/Hk .. (j+1)*Hq/Hk - 1)."""
    B, H, S, D = q.shape
    Hk = k.shape[1]
    if (k.shape != (B, Hk, S, D) or v.shape != k.shape or out.shape != q.shape or dout.shape != q.shape
            or Hk <= 0 or H % Hk):
        raise ValueError("attention_bwd needs q, out, dout [B, Hq, S, D] and k, v [B, Hk, S, D] with Hq % Hk == 0")
    if lse.shape != (B, H, S) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError("lse must be contiguous fp32 [B, H, S]")
    ts, strides = [], []
    for t, name in ((q, "q"), (k, "k"), (v, "v"), (out, "out"), (dout, "dout")):
        t, st = _bsh_strides(t, name)
        ts.append(t)
        strides += list(st)
    dev = q.device
    grads = [torch.empty(B, S, H, D, dtype=torch.bfloat16, device=dev).transpose(1, 2) for _ in range(3)]
    for g in grads:
        strides += [g.stride(0), g.stride(2), g.stride(1)]
    ws_bytes = lib().vq_attention_bwd_workspace(B, S, H)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(D)
    _check(lib().vq_attention_bwd(*(t.data_ptr() for t in ts), lse.data_ptr(), *(g.data_ptr() for g in grads), B, S,
                                  H, Hk, D, (ctypes.c_int64 * 24)(*strides), sc, ws.data_ptr(), ws.numel(),
                                  _stream(dev)),
           "vq_attention_bwd")
    return tuple(grads)


def swiglu_fwd(gu: torch.Tensor) -> torch.Tensor:
    t, f2 = gu.shape
    out = torch.empty(t, f2 // 2, dtype=torch.bfloat16, device=gu.device)
    _check(lib().vq_swiglu_fwd(_dev_ptr(gu, "gu"), t, f2 // 2, _dev_ptr(out, "out"), _stream(gu.device)),
           "vq_swiglu_fwd")
    return out


def swiglu_bwd(gu: torch.Tensor, dy: torch.Tensor) -> torch.Tensor:
    t, f2 = gu.shape
    dgu = torch.empty_like(gu)
    _check(lib().vq_swiglu_bwd(_dev_ptr(gu, "gu"), _dev_ptr(dy, "dy"), t, f2 // 2, _dev_ptr(dgu, "dgu"),
                               _stream(gu.device)),
           "vq_swiglu_bwd")
    return dgu


def add_rmsnorm_fwd(h: torch.Tensor, a: torch.Tensor | None, w: torch.Tensor, eps: float,
                    need_backward: bool = True):
    """(s, n, rstd): s = h + a (None when a is None), n = rms_norm(s) * w,
    rstd fp32 [rows] (None without a backward).  h, a: [rows, dim] bf16."""
    rows, dim = h.shape
    s = torch.empty_like(h) if a is not None else None
    n = torch.empty_like(h)
    rstd = torch.empty(rows, dtype=torch.float32, device=h.device) if need_backward else None
    _check(lib().vq_add_rmsnorm_fwd(_dev_ptr(h, "h"), _dev_ptr(a, "a"), _dev_ptr(w, "w"), rows, dim, float(eps),
                                    _dev_ptr(s, "s"), _dev_ptr(n, "n"), _dev_ptr(rstd, "rstd"), _stream(h.device)),
           "vq_add_rmsnorm_fwd")
    return s, n, rstd


def rmsnorm_bwd(dn: torch.Tensor, ds: torch.Tensor | None, s: torch.Tensor, w: torch.Tensor,
                rstd: torch.Tensor) -> torch.Tensor:
    rows, dim = s.shape
    dh = torch.empty_like(s)
    _check(lib().vq_rmsnorm_bwd(_dev_ptr(dn, "dn"), _dev_ptr(ds, "ds"), _dev_ptr(s, "s"), _dev_ptr(w, "w"),
                                _dev_ptr(rstd, "rstd"), rows, dim, _dev_ptr(dh, "dh"), _stream(s.device)),
           "vq_rmsnorm_bwd")
    return dh


def distill_loss_fwd(logits: torch.Tensor, teacher_logits: torch.Tensor, labels: torch.Tensor,
                     temperature: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(out fp32 [2] = (CE mean, KL mean), workspace for the backward)."""
    rows, vocab = logits.shape
    if logits.dtype != torch.bfloat16 or teacher_logits.dtype != torch.bfloat16:
        raise ValueError("logits must be bf16")
    if tuple(teacher_logits.shape) != (rows, vocab) or labels.numel() != rows or labels.dtype != torch.int64:
        raise ValueError("teacher_logits [rows, vocab] bf16 and labels [rows] int64 expected")
    dev = logits.device
    ws = torch.empty(max(int(lib().vq_distill_loss_workspace(rows)), 1), dtype=torch.uint8, device=dev)
    out = torch.empty(2, dtype=torch.float32, device=dev)
    _check(lib().vq_distill_loss_fwd(_dev_ptr(logits, "logits"), _dev_ptr(teacher_logits, "teacher_logits"),
                                     _dev_ptr(labels, "labels"), rows, vocab, float(temperature), _dev_ptr(out, "out"),
                                     _dev_ptr(ws, "workspace"), ws.numel(), _stream(dev)),
           "vq_distill_loss_fwd")
    return out, ws


def distill_loss_bwd(logits: torch.Tensor, teacher_logits: torch.Tensor, labels: torch.Tensor, temperature: float,
                     grad_out: torch.Tensor, ws: torch.Tensor) -> torch.Tensor:
    rows, vocab = logits.shape
    dev = logits.device
    g = torch.empty_like(logits)
    _check(lib().vq_distill_loss_bwd(_dev_ptr(logits, "logits"), _dev_ptr(teacher_logits, "teacher_logits"),
                                     _dev_ptr(labels, "labels"), rows, vocab, float(temperature),
                                     _dev_ptr(grad_out, "grad_out"), _dev_ptr(g, "grad_logits"),
                                     _dev_ptr(ws, "workspace"), ws.numel(), _stream(dev)),
           "vq_distill_loss_bwd")
    return g


def gated_linear_fwd(x: torch.Tensor, ggml_types, qbytes, probs: torch.Tensor, n: int, d_pad: int,
                     w_eff: torch.Tensor, y: torch.Tensor, workspace: torch.Tensor | None = None) -> None:
    """workspace: optional uint8 tensor of fwd_workspace_bytes(m, n, d) (lets the
    GEMM split its last round of tiles along K)."""
    m, d = x.shape
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check(lib().vq_gated_linear_fwd(_dev_ptr(x, "x"), m, n, d, d_pad, len(ggml_types), _int_array(ggml_types),
                                     _ptr_array(qbytes, "qbytes"), _dev_ptr(probs, "probs"),
                                     _dev_ptr(w_eff, "w_eff"), _dev_ptr(y, "y"), _dev_ptr(workspace, "workspace"),
                                     ws_bytes, _stream(x.device)),
           "vq_gated_linear_fwd")


def bwd_workspace_bytes(m: int, n: int, d: int, d_pad: int, ncand: int, need_w_eff: bool) -> int:
    v = int(lib().vq_gated_linear_bwd_workspace(m, n, d, d_pad, ncand, int(need_w_eff)))
    if v < 0:
        raise ValueError(f"invalid backward sizes m={m} n={n} d={d} ncand={ncand}")
    return v


def gated_linear_bwd(dy: torch.Tensor, x: torch.Tensor, ggml_types, qbytes, probs: torch.Tensor | None, n: int,
                     d_pad: int, w_eff: torch.Tensor | None, dx: torch.Tensor | None,
                     dprobs: torch.Tensor | None, workspace: torch.Tensor | None,
                     gate_stream: torch.cuda.Stream | None = None) -> None:
    """gate_stream: finish the gate gradient (dot pass, reduce into dprobs)
    on that stream, after a fence on the current one."""
    m, d = x.shape
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    args = (_dev_ptr(dy, "dy"), _dev_ptr(x, "x"), m, n, d, d_pad, len(ggml_types), _int_array(ggml_types),
            _ptr_array(qbytes, "qbytes"), _dev_ptr(probs, "probs"), _dev_ptr(w_eff, "w_eff"), _dev_ptr(dx, "dx"),
            _dev_ptr(dprobs, "dprobs"), _dev_ptr(workspace, "workspace"), ws_bytes, _stream(dy.device))
    if gate_stream is None:
        _check(lib().vq_gated_linear_bwd(*args), "vq_gated_linear_bwd")
    else:
        _check(lib().vq_gated_linear_bwd_gate_stream(*args, gate_stream.cuda_stream),
               "vq_gated_linear_bwd_gate_stream")


def fused_workspace_bytes(m: int, n: int, d: int, dx: bool) -> int:
    v = int(lib().vq_gated_linear_fused_workspace(m, n, d, int(dx)))
    if v < 0:
        raise ValueError(f"invalid fused sizes m={m} n={n} d={d}")
    return v


def _fused(entry: str, act: torch.Tensor, ggml_types, qbytes, probs: torch.Tensor, n: int, d: int, d_pad: int,
           out: torch.Tensor, workspace: torch.Tensor | None) -> None:
    m = act.shape[0]
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check(getattr(lib(), entry)(_dev_ptr(act, "activations"), m, n, d, d_pad, len(ggml_types),
                                 _int_array(ggml_types), _ptr_array(qbytes, "qbytes"), _dev_ptr(probs, "probs"),
                                 _dev_ptr(out, "out"), _dev_ptr(workspace, "workspace"), ws_bytes,
                                 _stream(act.device)),
           entry)


def gated_linear_fwd_fused(x: torch.Tensor, ggml_types, qbytes, probs: torch.Tensor, n: int, d_pad: int,
                           y: torch.Tensor, workspace: torch.Tensor | None = None) -> None:
    """y [m, n] = x @ W_eff^T with W_eff built in LDS (never in memory)."""
    _fused("vq_gated_linear_fwd_fused", x, ggml_types, qbytes, probs, n, x.shape[1], d_pad, y, workspace)


def gated_linear_dx_fused(dy: torch.Tensor, ggml_types, qbytes, probs: torch.Tensor, d: int, d_pad: int,
                          dx: torch.Tensor, workspace: torch.Tensor | None = None) -> None:
    """dx [m, d] = dy @ W_eff with W_eff built in LDS (never in memory)."""
    _fused("vq_gated_linear_dx_fused", dy, ggml_types, qbytes, probs, dy.shape[1], d, d_pad, dx, workspace)


STATIC_SCRATCH_BYTES = 4 << 20  # VQ_STATIC_SCRATCH_BYTES of include/voodoo_hip.h


def gated_linear_bwd_static(dy: torch.Tensor, x: torch.Tensor, ggml_types, qbytes, n: int, d_pad: int,
                            w_eff: torch.Tensor | None, dx: torch.Tensor | None,
                            dprobs: torch.Tensor | None) -> None:
    """The backward without a workspace: the library's static per-device
    scratch holds the gate partials (no allocation; overlapping calls on one
    device race)."""
    m, d = x.shape
    _check(lib().vq_gated_linear_bwd_static(_dev_ptr(dy, "dy"), _dev_ptr(x, "x"), m, n, d, d_pad, len(ggml_types),
                                            _int_array(ggml_types), _ptr_array(qbytes, "qbytes"),
                                            _dev_ptr(w_eff, "w_eff"), _dev_ptr(dx, "dx"), _dev_ptr(dprobs, "dprobs"),
                                            _stream(dy.device)),
           "vq_gated_linear_bwd_static")
