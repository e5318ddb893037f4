"""Tensor-level wrappers over the C ABI (one function per entry point).

Every function enqueues on the current torch stream of the tensors' device,
allocates its outputs with the torch caching allocator, validates shapes with
the exception types the reference uses (AssertionError for shape contracts,
TypeError/RuntimeError otherwise) and never falls back to a CPU path.
"""
import torch

from . import _hip


def _rows_view(x: torch.Tensor, width: int):
    """Return (tensor, rows, row_stride) for x viewed as [rows, width] with a
    unit inner stride, copying only if that view does not exist."""
    if x.dim() == 1:
        x = x.unsqueeze(0)
    if x.stride(-1) != 1:
        x = x.contiguous()
    lead = x.shape[:-1]
    rows = 1
    for d in lead:
        rows *= d
    if x.shape[-1] < width:
        raise AssertionError(f"last dimension {x.shape[-1]} < required {width}")
    if x.dim() == 2:
        return x, rows, x.stride(0)
    # collapsible leading dims with uniform row stride?
    ok = True
    expect = x.stride(-2)
    for i in range(x.dim() - 2, -1, -1):
        if x.shape[i] != 1 and x.stride(i) != expect:
            ok = False
            break
        expect *= x.shape[i]
    if not ok:
        x = x.contiguous()
        return x, rows, x.stride(-2)
    return x, rows, x.stride(-2) if rows > 1 else width


# ------------------------------------------------------------------ ternary

def ternary_gamma(w: torch.Tensor) -> torch.Tensor:
    """gamma = mean(|w|) + 1e-8 as a 1-element float32 device tensor
    (physics.py:24), deterministic float64 reduction."""
    _hip.require_device(w, "weight")
    w = w.detach().float().contiguous()
    g = torch.empty(1, device=w.device, dtype=torch.float32)
    _hip.call("walsh_ternary_gamma", w.data_ptr(), w.numel(), g.data_ptr(), _hip.stream(w.device))
    return g


def ternary_quantize(w: torch.Tensor, gamma: torch.Tensor = None, codes=False, packed=True, scaled=False):
    """Absmean ternary quantisation of ``w`` viewed as [rows, K] (K = last dim).

    Returns dict with 'gamma' and the requested outputs: 'codes' int8 [.., K],
    'packed' uint8 [.., ceil(K/4)] (pack_ternary_weights layout, fht_cuda.py:65-93),
    'scaled' float32 [.., K] = code*gamma (moe.py:288)."""
    _hip.require_device(w, "weight")
    w = w.detach().float().contiguous()
    K = w.shape[-1]
    rows = w.numel() // K
    if gamma is None:
        gamma = ternary_gamma(w)
    out = {"gamma": gamma}
    dev = w.device
    c = torch.empty(w.shape, device=dev, dtype=torch.int8) if codes else None
    p = torch.empty(w.shape[:-1] + ((K + 3) // 4,), device=dev, dtype=torch.uint8) if packed else None
    s = torch.empty(w.shape, device=dev, dtype=torch.float32) if scaled else None
    _hip.call("walsh_ternary_quantize", w.data_ptr(), rows, K, gamma.data_ptr(), _hip.ptr(c), _hip.ptr(p),
              _hip.ptr(s), _hip.stream(dev))
    if codes:
        out["codes"] = c
    if packed:
        out["packed"] = p
    if scaled:
        out["scaled"] = s
    return out


def ternary_unpack(packed: torch.Tensor, K: int) -> torch.Tensor:
    """int8 codes [.., K] from the 2-bit layout (fht_cuda.py:96-117)."""
    _hip.require_device(packed, "packed")
    packed = packed.contiguous()
    rows = packed.numel() // packed.shape[-1]
    assert packed.shape[-1] == (K + 3) // 4, "packed last dim must be ceil(K/4)"
    out = torch.empty(packed.shape[:-1] + (K,), device=packed.device, dtype=torch.int8)
    _hip.call("walsh_ternary_unpack", packed.data_ptr(), rows, K, out.data_ptr(), _hip.stream(packed.device))
    return out


# ------------------------------------------------------------------ hadamard

def hadamard_prepare(packed: torch.Tensor, in_o: int, out_o: int) -> torch.Tensor:
    """Kernel weight layout from packed codes [32, out_o, ceil(in_o/4)]."""
    _hip.require_device(packed, "packed weight")
    assert tuple(packed.shape) == (32, out_o, (in_o + 3) // 4), f"packed shape {tuple(packed.shape)}"
    n = _hip.lib().walsh_hadamard_weight_bytes(in_o, out_o)
    kw = torch.empty(n, device=packed.device, dtype=torch.uint8)
    _hip.call("walsh_hadamard_prepare", packed.contiguous().data_ptr(), in_o, out_o, kw.data_ptr(),
              _hip.stream(packed.device))
    return kw


def hadamard_linear(x: torch.Tensor, in_o: int, out_o: int, kweight: torch.Tensor, alpha: torch.Tensor,
                    beta: torch.Tensor, out_dtype: torch.dtype = None) -> torch.Tensor:
    """HadamardLinear forward (fht_cuda.py:489-519) on x [..., >=32*in_o].

    Computes in float32 matrix cores for float32 activations and bf16 matrix
    cores (float32 accumulate) for bfloat16 activations.  Returns
    [..., 32*out_o] in ``out_dtype`` (default x.dtype; must equal it)."""
    _hip.require_device(x, "input")
    dt = x.dtype if out_dtype is None else out_dtype
    if dt != x.dtype:
        x = x.to(dt)
    code = _hip.dtype_code(dt)
    C_in = 32 * in_o
    lead = x.shape[:-1]
    xv, rows, ldx = _rows_view(x, C_in)
    y = torch.empty(lead + (32 * out_o,), device=x.device, dtype=dt)
    if rows == 0:
        return y
    alpha = alpha.detach().float().contiguous()
    beta = beta.detach().float().contiguous()
    assert alpha.numel() == C_in and beta.numel() == 32 * out_o, "alpha/beta shapes"
    _hip.call("walsh_hadamard_linear_fwd", xv.data_ptr(), ldx, rows, in_o, out_o, kweight.data_ptr(),
              alpha.data_ptr(), beta.data_ptr(), y.data_ptr(), 32 * out_o, code, _hip.stream(x.device))
    return y
