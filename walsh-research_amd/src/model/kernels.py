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


def _had_meta(rows, in_o, out_o, dt, vec, kc1, swiglu=False):
    esz = 2 if dt == torch.bfloat16 else 4
    tag = "bf16" if dt == torch.bfloat16 else "f32"
    if swiglu:
        kname = "hadamard_swiglu_kernel<%s,%s>" % (tag, "vec" if vec else "scalar")
        nbytes = rows * 32 * (in_o + out_o) * esz + 2 * 32 * out_o * ((in_o + 3) // 4) + 8 * 32 * (in_o + out_o)
        flops = rows * 2 * (2 * 32 * in_o * out_o + 10 * 32 * (in_o + out_o)) + rows * 32 * out_o * 4
    else:
        kname = "hadamard_fwd_kernel<%s,%s,%s>" % (tag, "vec" if vec else "scalar", "kc1" if kc1 else "kloop")
        nbytes = rows * 32 * (in_o + out_o) * esz + 32 * out_o * ((in_o + 3) // 4) + 4 * 32 * (in_o + out_o)
        flops = rows * (2 * 32 * in_o * out_o + 10 * 32 * (in_o + out_o) + 32 * (in_o + out_o))
    return kname, nbytes, flops


def hadamard_linear(x: torch.Tensor, in_o: int, out_o: int, kweight: torch.Tensor, alpha: torch.Tensor,
                    beta: torch.Tensor, out_dtype: torch.dtype = None, gsx: int = None,
                    gsy: int = None) -> torch.Tensor:
    """HadamardLinear forward (fht_cuda.py:489-519) on x [..., >=32*gsx].

    Computes in float32 matrix cores for float32 activations and bf16 matrix
    cores (float32 accumulate) for bfloat16 activations.  gsx / gsy are the
    group strides of the input and output rows (default in_o / out_o); the
    result is [..., 32*gsy] in ``out_dtype`` (default x.dtype; must equal it)."""
    _hip.require_device(x, "input")
    dt = x.dtype if out_dtype is None else out_dtype
    if dt != x.dtype:
        x = x.to(dt)
    code = _hip.dtype_code(dt)
    gsx = in_o if gsx is None else gsx
    gsy = out_o if gsy is None else gsy
    lead = x.shape[:-1]
    xv, rows, ldx = _rows_view(x, 32 * gsx)
    y = torch.empty(lead + (32 * gsy,), device=x.device, dtype=dt)
    if rows == 0:
        return y
    alpha = alpha.detach().float().contiguous()
    beta = beta.detach().float().contiguous()
    assert alpha.numel() == 32 * in_o and beta.numel() == 32 * out_o, "alpha/beta shapes"
    esz = x.element_size()
    vec = gsx % 4 == 0 and gsy % 4 == 0 and ldx % 4 == 0 and xv.data_ptr() % (4 * esz) == 0
    kc1 = in_o <= 16 and (dt == torch.bfloat16 or out_o <= 16)
    kname, nbytes, flops = _had_meta(rows, in_o, out_o, dt, vec, kc1)
    _hip.call("walsh_hadamard_linear_ex_fwd", xv.data_ptr(), ldx, gsx, rows, in_o, out_o, kweight.data_ptr(),
              alpha.data_ptr(), beta.data_ptr(), y.data_ptr(), 32 * gsy, gsy, code, _hip.stream(x.device),
              kernel=kname, nbytes=nbytes, flops=flops)
    return y


def hadamard_swiglu(x: torch.Tensor, in_o: int, hid_o: int, gate, up, gsh: int = None) -> torch.Tensor:
    """silu(gate(x)) * up(x) for two Hadamard linears (chassis.py:498-504);
    gate/up = (kweight, alpha, beta).  Returns [..., 32*gsh] with group stride
    gsh (default roundup(hid_o, 4); pad slots are zeros)."""
    _hip.require_device(x, "input")
    dt = x.dtype
    code = _hip.dtype_code(dt)
    gsh = ((hid_o + 3) // 4) * 4 if gsh is None else gsh
    lead = x.shape[:-1]
    xv, rows, ldx = _rows_view(x, 32 * in_o)
    h = torch.empty(lead + (32 * gsh,), device=x.device, dtype=dt)
    if rows == 0:
        return h
    kg, ag, bg = gate
    ku, au, bu = up
    ag, bg, au, bu = (t.detach().float().contiguous() for t in (ag, bg, au, bu))
    esz = x.element_size()
    vec = in_o % 4 == 0 and gsh % 4 == 0 and ldx % 4 == 0 and xv.data_ptr() % (4 * esz) == 0
    kname, nbytes, flops = _had_meta(rows, in_o, hid_o, dt, vec, True, swiglu=True)
    _hip.call("walsh_hadamard_swiglu_fwd", xv.data_ptr(), ldx, in_o, rows, in_o, hid_o, kg.data_ptr(), ag.data_ptr(),
              bg.data_ptr(), ku.data_ptr(), au.data_ptr(), bu.data_ptr(), h.data_ptr(), 32 * gsh, gsh, code,
              _hip.stream(x.device), kernel=kname, nbytes=nbytes, flops=flops)
    return h


def fht(x: torch.Tensor, normalize: bool = True) -> torch.Tensor:
    """Fast Walsh-Hadamard transform along the last dim (fht_cuda.py:281-309)."""
    _hip.require_device(x, "input")
    N = x.shape[-1]
    dt = x.dtype if x.dtype in (torch.float32, torch.bfloat16) else torch.float32
    xc = x.to(dt).contiguous()
    y = torch.empty_like(xc)
    rows = xc.numel() // N if N else 0
    _hip.call("walsh_fht_fwd", xc.data_ptr(), rows, N, int(bool(normalize)), y.data_ptr(), _hip.dtype_code(dt),
              _hip.stream(x.device))
    return y


# ------------------------------------------------------------------ octonion

def octonion_prepare(packed: torch.Tensor, in_o: int, out_o: int, dtype: torch.dtype) -> torch.Tensor:
    """Dense signed-permutation block matrix [8*out_o, Kp] (elements of dtype)
    from packed codes [8, out_o, ceil(in_o/4)]."""
    _hip.require_device(packed, "packed weight")
    assert tuple(packed.shape) == (8, out_o, (in_o + 3) // 4), f"packed shape {tuple(packed.shape)}"
    n = _hip.lib().walsh_octonion_weight_elems(in_o, out_o)
    B = torch.empty(n, device=packed.device, dtype=dtype)
    _hip.call("walsh_octonion_prepare", packed.contiguous().data_ptr(), in_o, out_o, B.data_ptr(),
              _hip.dtype_code(dtype), _hip.stream(packed.device))
    return B


def octonion_linear(x: torch.Tensor, in_o: int, out_o: int, B: torch.Tensor, beta: torch.Tensor) -> torch.Tensor:
    """Cayley-Dickson ternary linear on full rows x [..., 8*in_o] -> [..., 8*out_o]
    (physics.py:66-82); B from octonion_prepare in x.dtype."""
    _hip.require_device(x, "input")
    assert B.dtype == x.dtype, "prepared weight dtype must match the activation dtype"
    K = 8 * in_o
    lead = x.shape[:-1]
    xv, rows, ldx = _rows_view(x, K)
    y = torch.empty(lead + (8 * out_o,), device=x.device, dtype=x.dtype)
    if rows == 0:
        return y
    vec = 16 // x.element_size()
    if ldx % vec or xv.data_ptr() % 16:
        xv = xv.reshape(rows, -1)[:, :K].contiguous()
        ldx = K
    beta = beta.detach().float().contiguous()
    esz = x.element_size()
    nbytes = rows * 8 * (in_o + out_o) * esz + 8 * out_o * ((in_o + 3) // 4) + 4 * out_o
    flops = 2 * rows * (8 * in_o) * (8 * out_o)
    _hip.call("walsh_octonion_linear_fwd", xv.data_ptr(), ldx, rows, in_o, out_o, B.data_ptr(), beta.data_ptr(),
              y.data_ptr(), 8 * out_o, _hip.dtype_code(x.dtype), _hip.stream(x.device),
              kernel="octonion_gemm_kernel<%s>" % ("bf16" if x.dtype == torch.bfloat16 else "f32"),
              nbytes=nbytes, flops=flops)
    return y


# ------------------------------------------------------------------ mHC

def sinkhorn(h: torch.Tensor, n_iter: int = 20, eps: float = 1e-8) -> torch.Tensor:
    """SinkhornKnopp.forward (mhc.py:214-229) on [..., n, n] (computed in float32)."""
    _hip.require_device(h, "H")
    n = h.shape[-1]
    assert h.shape[-2] == n, "Sinkhorn needs square matrices"
    hf = h.detach().float().contiguous()
    out = torch.empty_like(hf)
    batch = hf.numel() // (n * n)
    _hip.call("walsh_sinkhorn_fwd", hf.data_ptr(), batch, n, int(n_iter), float(eps), out.data_ptr(),
              _hip.stream(h.device))
    return out


def mhc_pre(x: torch.Tensor, phi_cat: torch.Tensor, coef: torch.Tensor, bias_cat: torch.Tensor, rms_eps: float,
            n_iter: int = 20, sk_eps: float = 1e-8):
    """Fused mappings + H_pre @ x for x [..., n, C] (mhc.py:283-318, 345-364).

    phi_cat [32, n*C] in x.dtype (rows pre|post|res|0), coef float32 [3],
    bias_cat float32 [2n + n*n].  Returns (layer_in [..., C], H_pre [..., n],
    H_post [..., n], H_res [..., n, n]) with the H's in float32."""
    _hip.require_device(x, "stream input")
    n, C = x.shape[-2], x.shape[-1]
    lead = x.shape[:-2]
    xv = x if x.is_contiguous() else x.contiguous()
    M = xv.numel() // (n * C)
    dev = x.device
    layer_in = torch.empty(lead + (C,), device=dev, dtype=x.dtype)
    h_pre = torch.empty(lead + (n,), device=dev, dtype=torch.float32)
    h_post = torch.empty(lead + (n,), device=dev, dtype=torch.float32)
    h_res = torch.empty(lead + (n, n), device=dev, dtype=torch.float32)
    if M == 0:
        return layer_in, h_pre, h_post, h_res
    assert phi_cat.dtype == x.dtype and tuple(phi_cat.shape) == (32, n * C), "phi_cat layout"
    esz = x.element_size()
    nbytes = M * (n * C + C) * esz + M * (2 * n + n * n) * 4 + (2 * n + n * n) * n * C * esz
    flops = M * (2 * n * C * (2 * n + n * n) + 2 * n * C + 2 * n * C)
    _hip.call("walsh_mhc_pre_fwd", xv.data_ptr(), n * C, M, n, C, phi_cat.data_ptr(), coef.data_ptr(),
              bias_cat.data_ptr(), float(rms_eps), int(n_iter), float(sk_eps), h_pre.data_ptr(), h_post.data_ptr(),
              h_res.data_ptr(), layer_in.data_ptr(), C, _hip.dtype_code(x.dtype), _hip.stream(dev),
              kernel="mhc_pre_kernel<%s>" % ("bf16" if x.dtype == torch.bfloat16 else "f32"), nbytes=nbytes,
              flops=flops)
    return layer_in, h_pre, h_post, h_res


def phi_fragments(phi_cat: torch.Tensor) -> torch.Tensor:
    """phi_cat [32, K] -> matrix-core fragment order [K/16][2][64][4] (K % 16 == 0)."""
    K = phi_cat.shape[1]
    return phi_cat.view(2, 16, K // 16, 4, 4).permute(2, 0, 3, 1, 4).contiguous()


def mhc_pre_supported(n: int, C: int, dtype: torch.dtype) -> bool:
    """Whether walsh_mhc_pre_norm_fwd handles this shape (16 rows fit in LDS)."""
    esz = 2 if dtype == torch.bfloat16 else 4
    return n <= 4 and (n * C) % 16 == 0 and C % 4 == 0 and C <= 1024 and n * C * esz * 16 <= 128 * 1024


def mhc_pre_norm(x: torch.Tensor, phi_frag: torch.Tensor, coef: torch.Tensor, bias_cat: torch.Tensor,
                 rms_eps: float, norm_w: torch.Tensor = None, norm_eps: float = 1e-6, n_iter: int = 20,
                 sk_eps: float = 1e-8):
    """mhc_pre with the token tile held in LDS (one HBM pass over x) and the
    optional RMSNorm of layer_in fused (chassis.py:96-106)."""
    _hip.require_device(x, "stream input")
    n, C = x.shape[-2], x.shape[-1]
    lead = x.shape[:-2]
    xv = x if x.is_contiguous() else x.contiguous()
    M = xv.numel() // (n * C)
    dev = x.device
    layer_in = torch.empty(lead + (C,), device=dev, dtype=x.dtype)
    h_pre = torch.empty(lead + (n,), device=dev, dtype=torch.float32)
    h_post = torch.empty(lead + (n,), device=dev, dtype=torch.float32)
    h_res = torch.empty(lead + (n, n), device=dev, dtype=torch.float32)
    if M == 0:
        return layer_in, h_pre, h_post, h_res
    assert phi_frag.dtype == x.dtype and phi_frag.numel() == 32 * n * C, "phi_frag layout"
    nw = None
    if norm_w is not None:
        nw = norm_w.detach().float().contiguous()
        assert nw.numel() == C
    esz = x.element_size()
    nbytes = M * (n * C + C) * esz + M * (2 * n + n * n) * 4 + 32 * n * C * esz
    flops = M * (2 * n * C * 32 + 2 * n * C + 2 * n * C)
    _hip.call("walsh_mhc_pre_norm_fwd", xv.data_ptr(), n * C, M, n, C, phi_frag.data_ptr(), coef.data_ptr(),
              bias_cat.data_ptr(), float(rms_eps), int(n_iter), float(sk_eps), h_pre.data_ptr(), h_post.data_ptr(),
              h_res.data_ptr(), layer_in.data_ptr(), C, _hip.ptr(nw), float(norm_eps), _hip.dtype_code(x.dtype),
              _hip.stream(dev), kernel="mhc_pre2_kernel<%s>" % ("bf16" if x.dtype == torch.bfloat16 else "f32"),
              nbytes=nbytes, flops=flops)
    return layer_in, h_pre, h_post, h_res


def mhc_post(x: torch.Tensor, out: torch.Tensor, h_res: torch.Tensor, h_post: torch.Tensor) -> torch.Tensor:
    """x_new = H_res @ x + H_post^T (x) out (mhc.py:366-381); x [..., n, C], out [..., C]."""
    _hip.require_device(x, "stream input")
    n, C = x.shape[-2], x.shape[-1]
    xv = x if x.is_contiguous() else x.contiguous()
    M = xv.numel() // (n * C)
    o = out.to(x.dtype)
    o = o if o.is_contiguous() else o.contiguous()
    assert o.numel() == M * C, "layer output shape"
    x_new = torch.empty_like(xv)
    if M == 0:
        return x_new
    hr = h_res.detach().float().contiguous()
    hp = h_post.detach().float().contiguous()
    esz = x.element_size()
    nbytes = M * (2 * n * C + C) * esz + M * (n * n + n) * 4
    flops = M * n * C * (2 * n + 2)
    _hip.call("walsh_mhc_post_fwd", xv.data_ptr(), n * C, o.data_ptr(), C, hr.data_ptr(), hp.data_ptr(),
              x_new.data_ptr(), n * C, M, n, C, _hip.dtype_code(x.dtype), _hip.stream(x.device),
              kernel="mhc_post_kernel<%s>" % ("bf16" if x.dtype == torch.bfloat16 else "f32"), nbytes=nbytes,
              flops=flops)
    return x_new
