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


def ternary_ste_bwd(grad: torch.Tensor, w: torch.Tensor = None, mode: int = 1) -> torch.Tensor:
    """Straight-through gradient of the ternary quantisers: mode 1 clamps to
    [-2, 2] (TernaryAbsmeanSTE.backward, physics.py:35-39, moe.py:289-294);
    mode 0 passes the gradient where -1.5 <= w <= 1.5 (quantize_ternary's
    clamp path, physics.py:48-50).  float32, grad's shape."""
    _hip.require_device(grad, "gradient")
    g = grad.float().contiguous()
    out = torch.empty_like(g)
    wp = 0
    if mode == 0:
        assert w is not None and w.numel() == g.numel(), "mode 0 needs the latent weights"
        wf = w.detach().float().contiguous()
        wp = wf.data_ptr()
    _hip.call("walsh_ternary_ste_bwd", g.data_ptr(), wp, g.numel(), int(mode), out.data_ptr(), _hip.stream(g.device))
    return out


def ternary_from_bitmask(bitmask: torch.Tensor, sign_bits: torch.Tensor, num_nonzero: int, shape,
                         packed: bool = True, codes: bool = False) -> dict:
    """Decode a .walsh v4 bitmask + sign tensor (uint8 device buffers) on
    the GPU into the 2-bit packed layout [.., ceil(K/4)] and/or int8 codes of
    ``shape`` (generate_compressed.py:70-105 semantics)."""
    _hip.require_device(bitmask, "bitmask")
    shape = tuple(int(d) for d in shape)
    K = shape[-1]
    rows = 1
    for d in shape[:-1]:
        rows *= d
    dev = bitmask.device
    out = {}
    pk = torch.empty(shape[:-1] + ((K + 3) // 4,), device=dev, dtype=torch.uint8) if packed else None
    cd = torch.empty(shape, device=dev, dtype=torch.int8) if codes else None
    nws = _hip.lib().walsh_bitmask_workspace_bytes(rows * K)
    ws = torch.empty(max(nws, 4), device=dev, dtype=torch.uint8)
    bm = bitmask.contiguous()
    sg = sign_bits.contiguous()
    _hip.call("walsh_ternary_from_bitmask", bm.data_ptr() if bm.numel() else 0, bm.numel(),
              sg.data_ptr() if sg.numel() else 0, sg.numel(), int(num_nonzero), rows, K,
              0 if pk is None else pk.data_ptr(), 0 if cd is None else cd.data_ptr(), ws.data_ptr(), nws,
              _hip.stream(dev), kernel="bitmask_decode", nbytes=bm.numel() + sg.numel() + rows * ((K + 3) // 4))
    if pk is not None:
        out["packed"] = pk
    if cd is not None:
        out["codes"] = cd
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


# 16-row tiles per layer up to which the library runs the bf16 single-output-tile
# shapes on wavefront pairs (hadamard_pair_kernel / hadamard_pair_kpar_kernel);
# 16x16 layers on contiguous 512-value rows switch to the one-wavefront kernel
# (whole rows through LDS) above PAIR_MAX_TILES_ROWS
PAIR_MAX_TILES = 2048
PAIR_MAX_TILES_ROWS = 1024


def _whole_rows(in_o, out_o, ldx, dt, ptr):
    """16x16 bf16 layer on 16-byte aligned rows of 512 contiguous values
    (outputs allocated contiguous): the library's whole-row variant of the
    one-wavefront kernel."""
    return dt == torch.bfloat16 and in_o == 16 and out_o == 16 and ldx == 512 and ptr % 16 == 0


def _pair_shape(rows, in_o, out_o, dt, vec, rope=False, whole_rows=False):
    """The pair kernel the library dispatches for this shape, or None."""
    limit = PAIR_MAX_TILES_ROWS if whole_rows else PAIR_MAX_TILES
    if dt != torch.bfloat16 or not vec or out_o > 16 or (rows + 15) // 16 > limit:
        return None
    if in_o <= 16:
        return "hadamard_pair_kernel"
    if in_o <= 64 and not rope:
        return "hadamard_pair_kpar_kernel"
    return None


def _had_meta(rows, in_o, out_o, dt, vec, kc1, swiglu=False, rope=False, whole_rows=False):
    esz = 2 if dt == torch.bfloat16 else 4
    tag = "bf16" if dt == torch.bfloat16 else "f32"
    if swiglu:
        kname = "hadamard_swiglu_kernel<%s,%s>" % (tag, "vec" if vec else "scalar")
        nbytes = rows * 32 * (in_o + out_o) * esz + 2 * 32 * out_o * ((in_o + 3) // 4) + 8 * 32 * (in_o + out_o)
        flops = rows * 2 * (2 * 32 * in_o * out_o + 10 * 32 * (in_o + out_o)) + rows * 32 * out_o * 4
    else:
        pair = _pair_shape(rows, in_o, out_o, dt, vec, rope, whole_rows)
        kname = ("%s<%s>" % (pair, tag)) if pair else \
            "hadamard_fwd_kernel<%s,%s,%s>" % (tag, "vec" if vec else "scalar", "kc1" if kc1 else "kloop")
        if whole_rows and not pair:
            kname = "hadamard_fwd_kernel<bf16,rows>"
        nbytes = rows * 32 * (in_o + out_o) * esz + 32 * out_o * ((in_o + 3) // 4) + 4 * 32 * (in_o + out_o)
        flops = rows * (2 * 32 * in_o * out_o + 10 * 32 * (in_o + out_o) + 32 * (in_o + out_o))
    return kname, nbytes, flops


def rope_supported(x: torch.Tensor, out_o: int, head_dim: int) -> bool:
    """Can the rotary embedding ride on a Hadamard linear's store?"""
    return (x.is_cuda and head_dim >= 4 and head_dim % 4 == 0 and out_o % head_dim == 0
            and x.shape[-1] % 4 == 0 and x.stride(-1) == 1)


# The bf16 Hadamard kernels for in_o > 16 and out_o > 48 (n_embd 4096: the
# base-3 wide kernel and its decode-sized split) keep alpha and beta in LDS as
# float16 for the whole launch.  float16 overflows above 65504 and rounds
# non-zeros below 2^-24 (its smallest subnormal) to zero or to a value 100%
# off; in between, its absolute error stays below 2^-25 (relative 2^-11 from
# 2^-14 up, and no worse than the bf16 activations' 2^-8 down to 2^-16).  A
# value that float16 would destroy (a trained scale that blew up or collapsed,
# or a non-finite one) raises instead of being damaged silently.  The check
# reads the values once per parameter version (one host round trip after
# each optimizer step, none under graph capture).
F16_MAX = 65504.0
F16_MIN_SUBNORMAL = 2.0 ** -24
_f16_checked = {}


def half_scales_used(dtype: torch.dtype, in_o: int, out_o: int) -> bool:
    return dtype == torch.bfloat16 and 16 < in_o <= 128 and 48 < out_o <= 128


def check_half_range(name: str, t: torch.Tensor, scale: float = 1.0) -> None:
    """Raise ValueError if a value of ``t * scale`` is not finite, exceeds
    float16's largest value, or is a non-zero below its smallest subnormal.
    Cached on the tensor's storage and version."""
    if t is None or t.numel() == 0 or (t.is_cuda and torch.cuda.is_current_stream_capturing()):
        return
    key = (t.data_ptr(), t._version, t.numel(), scale)
    if key in _f16_checked:
        return
    a = t.detach().float().abs() * scale
    hi = float(a.max())
    nz = a[a > 0]
    lo = float(nz.min()) if nz.numel() else 1.0
    if not (hi <= F16_MAX) or lo < F16_MIN_SUBNORMAL:
        raise ValueError(f"{name}: |values| span [{lo:.3e}, {hi:.3e}], outside [{F16_MIN_SUBNORMAL:.3e}, {F16_MAX}]: "
                         f"the n_embd-4096 bf16 Hadamard kernels hold them as float16")
    if len(_f16_checked) > 4096:
        _f16_checked.clear()
    _f16_checked[key] = True


def hadamard_linear_rope(x: torch.Tensor, in_o: int, out_o: int, kweight: torch.Tensor, alpha: torch.Tensor,
                         beta: torch.Tensor, freqs_cis: torch.Tensor, head_dim: int) -> torch.Tensor:
    """HadamardLinear forward followed by apply_rotary_emb (chassis.py:339-345)
    on x [B, T, C]: row (b, t) turns by freqs_cis[t] (complex [T, head_dim/2])."""
    _hip.require_device(x, "input")
    dt = x.dtype
    B, T = x.shape[0], x.shape[1]
    xv, rows, ldx = _rows_view(x, 32 * in_o)
    if xv.data_ptr() % (4 * x.element_size()) or ldx % 4:
        xv = xv.contiguous()
        ldx = xv.stride(0)
    y = torch.empty(x.shape[:-1] + (32 * out_o,), device=x.device, dtype=dt)
    if rows == 0:
        return y
    table = torch.view_as_real(freqs_cis[:T].contiguous())
    assert table.shape == (T, head_dim // 2, 2) and table.dtype == torch.float32, "freqs_cis shape"
    if half_scales_used(dt, in_o, out_o):
        check_half_range("alpha", alpha)
        check_half_range("beta", beta)
    alpha = alpha.detach().float().contiguous()
    beta = beta.detach().float().contiguous()
    vec = True
    kc1 = in_o <= 16
    kname, nbytes, flops = _had_meta(rows, in_o, out_o, dt, vec, kc1, rope=True,
                                     whole_rows=_whole_rows(in_o, out_o, ldx, dt, xv.data_ptr()))
    if in_o > 16 and out_o > 48:
        kname = "hadamard_wide3_kernel<bf16>" if dt == torch.bfloat16 and in_o <= 128 and out_o <= 128 else \
            "hadamard_wide_kernel<%s>" % ("bf16" if dt == torch.bfloat16 else "f32")
    _hip.call("walsh_hadamard_linear_rope_fwd", xv.data_ptr(), ldx, rows, in_o, out_o, kweight.data_ptr(),
              alpha.data_ptr(), beta.data_ptr(), table.data_ptr(), T, head_dim, y.data_ptr(), 32 * out_o,
              _hip.dtype_code(dt), _hip.stream(x.device), kernel=kname, nbytes=nbytes, flops=flops)
    return y


def _group_rows_view(y: torch.Tensor, rows: int, out_o: int):
    """(row stride, group stride) of an output given as [rows, 32, out_o]
    (any leading shape with that many rows) with unit inner stride, or None."""
    if y.dim() < 2 or y.stride(-1) != 1 or y.shape[-1] != out_o or y.shape[-2] != 32:
        return None
    lead = [(d, st) for d, st in zip(y.shape[:-2], y.stride()[:-2]) if d != 1]
    if len(lead) > 1 or (lead and lead[0][0] != rows) or (not lead and rows != 1):
        return None
    return (lead[0][1] if lead else 32 * y.stride(-2)), y.stride(-2)


def hadamard_linear_multi(x: torch.Tensor, in_o: int, out_o: int, layers, freqs_cis: torch.Tensor = None,
                          head_dim: int = None, outs=None):
    """Several Hadamard linears of one shape on the same rows x [B, T, C] in
    one launch: ``layers`` = [(kweight, alpha, beta, rope)], rope True applies
    the rotary embedding (freqs_cis rows, head_dim) on that layer's store.
    Returns the outputs [B, T, 32*out_o] in x.dtype.  ``outs`` may give, per
    layer, a tensor to write instead (None: allocate), viewed as
    [rows, 32, out_o] with any row and group strides (e.g. a KV cache slot
    [B, 1, n_head, head_dim]); it is returned in that layer's place."""
    import ctypes
    _hip.require_device(x, "input")
    n = len(layers)
    dt = x.dtype
    B, T = x.shape[0], x.shape[1]
    xv, rows, ldx = _rows_view(x, 32 * in_o)
    if xv.data_ptr() % (4 * x.element_size()) or ldx % 4:
        xv = xv.contiguous()
        ldx = xv.stride(0)
    outs = list(outs) if outs is not None else [None] * n
    ys = [o if o is not None else torch.empty(x.shape[:-1] + (32 * out_o,), device=x.device, dtype=dt)
          for o in outs]
    if rows == 0:
        return ys
    strides = []
    for i, o in enumerate(outs):
        if o is None:
            strides.append((32 * out_o, out_o))
        else:
            st = _group_rows_view(o, rows, out_o)
            assert st is not None and o.dtype == dt, "output view must be [rows, 32, out_o] in x.dtype"
            strides.append(st)
    keep = []
    kws, als, bes, yps = [], [], [], []
    mask = 0
    for i, (kw, a, b, rope) in enumerate(layers):
        if half_scales_used(dt, in_o, out_o):
            check_half_range("alpha", a)
            check_half_range("beta", b)
        a = a.detach().float().contiguous()
        b = b.detach().float().contiguous()
        keep += [a, b]
        kws.append(kw.data_ptr())
        als.append(a.data_ptr())
        bes.append(b.data_ptr())
        yps.append(ys[i].data_ptr())
        mask |= (1 << i) if rope else 0
    table = None
    if mask:
        table = torch.view_as_real(freqs_cis[:T].contiguous())
        assert table.shape == (T, head_dim // 2, 2) and table.dtype == torch.float32, "freqs_cis shape"
    arrs = [(ctypes.c_void_p * n)(*v) for v in (kws, als, bes, yps)]
    kname, nbytes, flops = _had_meta(rows, in_o, out_o, dt, True, in_o <= 16)
    nbytes = rows * 32 * (in_o + n * out_o) * x.element_size()
    whole = _whole_rows(in_o, out_o, ldx, dt, xv.data_ptr()) and all(o is None for o in outs)
    kname = ("hadamard_pair_kernel<bf16,x%d>" % n) \
        if _pair_shape(rows, in_o, out_o, dt, True, whole_rows=whole) == "hadamard_pair_kernel" \
        else "hadamard_fwdn_kernel<%s,x%d%s>" % ("bf16" if dt == torch.bfloat16 else "f32", n, ",rows" if whole else "")
    rope_args = (0 if table is None else table.data_ptr(), T, head_dim or 4, mask, _hip.dtype_code(dt),
                 _hip.stream(x.device))
    if all(o is None for o in outs):
        _hip.call("walsh_hadamard_linear_multi_fwd", xv.data_ptr(), ldx, rows, in_o, out_o, n,
                  *[ctypes.addressof(a) for a in arrs], 32 * out_o, *rope_args, kernel=kname, nbytes=nbytes,
                  flops=flops * n)
    else:
        lds = (ctypes.c_int64 * n)(*[st[0] for st in strides])
        gss = (ctypes.c_int64 * n)(*[st[1] for st in strides])
        _hip.call("walsh_hadamard_linear_multi_ex_fwd", xv.data_ptr(), ldx, rows, in_o, out_o, n,
                  *[ctypes.addressof(a) for a in arrs], ctypes.addressof(lds), ctypes.addressof(gss), *rope_args,
                  kernel=kname, nbytes=nbytes, flops=flops * n)
    return ys


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
    if half_scales_used(dt, in_o, out_o):
        check_half_range("alpha", alpha)
        check_half_range("beta", beta)
    alpha = alpha.detach().float().contiguous()
    beta = beta.detach().float().contiguous()
    assert alpha.numel() == 32 * in_o and beta.numel() == 32 * out_o, "alpha/beta shapes"
    esz = x.element_size()
    vec = gsx % 4 == 0 and gsy % 4 == 0 and ldx % 4 == 0 and xv.data_ptr() % (4 * esz) == 0
    kc1 = in_o <= 16 and (dt == torch.bfloat16 or out_o <= 16)
    whole = gsx == 16 and gsy == 16 and _whole_rows(in_o, out_o, ldx, dt, xv.data_ptr())
    kname, nbytes, flops = _had_meta(rows, in_o, out_o, dt, vec, kc1, whole_rows=whole)
    if vec and in_o > 16 and out_o > 48:
        if dt == torch.bfloat16 and in_o <= 128 and out_o <= 128:
            kname = "hadamard_wide3_kernel<bf16>"
        else:
            kname = "hadamard_wide_kernel<%s>" % ("bf16" if dt == torch.bfloat16 else "f32")
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


def hadamard_mlp_supported(x: torch.Tensor, in_o: int, hid_o: int, out_o: int) -> bool:
    """Shapes of walsh_hadamard_mlp_fwd: bf16 rows, in_o and out_o <= 16
    (multiples of 4), 16 < hid_o <= 48."""
    return (x.is_cuda and x.dtype == torch.bfloat16 and 0 < in_o <= 16 and in_o % 4 == 0 and 16 < hid_o <= 48
            and 0 < out_o <= 16 and out_o % 4 == 0 and x.shape[-1] == 32 * in_o)


def hadamard_mlp(x: torch.Tensor, in_o: int, hid_o: int, out_o: int, gate, up, down) -> torch.Tensor:
    """down(silu(gate(x)) * up(x)) for three Hadamard linears (chassis.py:498-504)
    in one launch; gate/up/down = (kweight, alpha, beta).  Returns
    [..., 32*out_o] in x.dtype, bitwise equal to hadamard_swiglu followed by
    the down projection."""
    _hip.require_device(x, "input")
    assert hadamard_mlp_supported(x, in_o, hid_o, out_o), "hadamard_mlp shape"
    lead = x.shape[:-1]
    xv, rows, ldx = _rows_view(x, 32 * in_o)
    if xv.data_ptr() % 8 or ldx % 4:
        xv = xv.contiguous()
        ldx = xv.stride(0)
    y = torch.empty(lead + (32 * out_o,), device=x.device, dtype=x.dtype)
    if rows == 0:
        return y
    ws = []
    for kw, a, b in (gate, up, down):
        ws += [kw, a.detach().float().contiguous(), b.detach().float().contiguous()]
    gsh = (hid_o + 3) // 4 * 4
    nbytes = rows * 32 * (in_o + out_o) * 2 + 32 * (2 * hid_o * ((in_o + 3) // 4) + out_o * ((hid_o + 3) // 4))
    flops = rows * (2 * (2 * 32 * in_o * hid_o + 10 * 32 * (in_o + hid_o)) + 32 * hid_o * 4
                    + 2 * 32 * gsh * out_o + 10 * 32 * (gsh + out_o))
    _hip.call("walsh_hadamard_mlp_fwd", xv.data_ptr(), ldx, rows, in_o, hid_o, out_o,
              *[w.data_ptr() for w in ws], y.data_ptr(), 32 * out_o, _hip.dtype_code(x.dtype),
              _hip.stream(x.device), kernel="hadamard_mlp_kernel<bf16>", nbytes=nbytes, flops=flops)
    return y


def hadamard_pack_transpose(packed: torch.Tensor, in_o: int, out_o: int) -> torch.Tensor:
    """Packed codes of the transposed layer: [32, in_o, ceil(out_o/4)] from
    [32, out_o, ceil(in_o/4)] (fht_cuda.py:65-93 packing of W^T)."""
    _hip.require_device(packed, "packed weight")
    assert tuple(packed.shape) == (32, out_o, (in_o + 3) // 4), f"packed shape {tuple(packed.shape)}"
    pt = torch.empty(32, in_o, (out_o + 3) // 4, device=packed.device, dtype=torch.uint8)
    _hip.call("walsh_hadamard_pack_transpose", packed.contiguous().data_ptr(), in_o, out_o, pt.data_ptr(),
              _hip.stream(packed.device))
    return pt


def hadamard_prepare_t(packed: torch.Tensor, in_o: int, out_o: int) -> torch.Tensor:
    """Kernel weight layout of the transposed layer (in_o <-> out_o), the
    weights of the input-gradient pass."""
    return hadamard_prepare(hadamard_pack_transpose(packed, in_o, out_o), out_o, in_o)


def hadamard_linear_bwd(x: torch.Tensor, gy: torch.Tensor, in_o: int, out_o: int, kweight: torch.Tensor,
                        kweight_t: torch.Tensor, alpha: torch.Tensor, beta: torch.Tensor,
                        latent: torch.Tensor = None, need=(True, True, True, True), gsx: int = None,
                        gsy: int = None):
    """Backward of hadamard_linear for the output gradient ``gy``.

    Returns (gx, dalpha, dbeta, dweight); entries not requested in ``need``
    (same order) are None.  gx has x's shape and dtype; the others are
    float32 [32, in_o], [32, out_o], [32, out_o, in_o].  With ``latent`` the
    weight gradient passes the straight-through estimator's clamp
    (physics.py:48-50): zero where |latent| > 1.5.  gsx / gsy are the group
    strides of x (and gx) and gy rows, as in hadamard_linear."""
    _hip.require_device(x, "input")
    _hip.require_device(gy, "output gradient")
    dt = x.dtype
    code = _hip.dtype_code(dt)
    gsx = in_o if gsx is None else gsx
    gsy = out_o if gsy is None else gsy
    assert gy.dtype == dt, f"gradient dtype {gy.dtype} != input dtype {dt}"
    assert x.shape[-1] == 32 * gsx and gy.shape[-1] == 32 * gsy, "x / gy widths"
    assert x.shape[:-1] == gy.shape[:-1], "x / gy leading shapes differ"
    xc = x.reshape(-1, 32 * gsx).contiguous()
    gc = gy.reshape(-1, 32 * gsy).contiguous()
    M = xc.shape[0]
    dev = x.device
    want_x, want_a, want_b, want_w = need
    # the kernel writes pad slots up to roundup(in_o, 4); wider pads start at zero
    gx = (torch.zeros_like(xc) if gsx > (in_o + 3) // 4 * 4 else torch.empty_like(xc)) if want_x else None
    da = torch.empty(32, in_o, device=dev, dtype=torch.float32) if want_a else None
    db = torch.empty(32, out_o, device=dev, dtype=torch.float32) if want_b else None
    dw = torch.empty(32, out_o, in_o, device=dev, dtype=torch.float32) if want_w else None
    nws = _hip.lib().walsh_hadamard_bwd_workspace_bytes(M, gsx, gsy, code)
    ws = torch.empty(max(nws, 1), device=dev, dtype=torch.uint8)
    alpha = alpha.detach().float().contiguous()
    beta = beta.detach().float().contiguous()
    lat = None
    if latent is not None and want_w:
        lat = latent.detach().float().contiguous()
        assert lat.shape == (32, out_o, in_o), "latent weight shape"
    ptr = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
    esz = x.element_size()
    # algorithmic: x and gy read once, gx written once (+ the parameters)
    nbytes = M * 32 * (2 * in_o + out_o) * esz + 4 * 32 * (in_o + out_o) * 3 + 4 * 32 * in_o * out_o * 2
    flops = M * 32 * (3 * 2 * in_o * out_o + 20 * (in_o + out_o))
    _hip.call("walsh_hadamard_linear_ex_bwd", xc.data_ptr(), 32 * gsx, gsx, gc.data_ptr(), 32 * gsy, gsy, M, in_o,
              out_o, ptr(kweight), ptr(kweight_t), alpha.data_ptr(), beta.data_ptr(), ptr(lat), ptr(gx), 32 * gsx,
              ptr(da), ptr(db), ptr(dw), code, ws.data_ptr(), nws, _hip.stream(dev),
              kernel="hadamard_linear_bwd<%s>" % ("bf16" if dt == torch.bfloat16 else "f32"), nbytes=nbytes,
              flops=flops)
    if gx is not None:
        gx = gx.view(x.shape)
    return gx, da, db, dw


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


# ------------------------------------------------------------------ head mixer

HEAD_MIXER_MAX_D = 32        # any dtype (weights resident in LDS)
HEAD_MIXER_MAX_D_BF16 = 128  # bf16 (weights streamed, the wide kernel)


def head_mixer_supported(D: int, dtype: torch.dtype) -> bool:
    return D <= HEAD_MIXER_MAX_D or (dtype == torch.bfloat16 and D <= HEAD_MIXER_MAX_D_BF16 and D % 4 == 0)


def head_mixer_prepare(W: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Matrix-core fragments of the head mixer's dense W [32, D, D] (applied as
    x @ W[h]) in ``dtype`` (bf16 or float32)."""
    _hip.require_device(W, "head mixer weight")
    assert W.dim() == 3 and W.shape[0] == 32 and W.shape[1] == W.shape[2], f"W shape {tuple(W.shape)}"
    D = W.shape[1]
    code = _hip.dtype_code(dtype)
    n = _hip.lib().walsh_hadamard_dense_weight_bytes(D, D, code)
    kw = torch.empty(n, device=W.device, dtype=torch.uint8)
    wf = W.detach().float().contiguous()
    _hip.call("walsh_hadamard_dense_prepare", wf.data_ptr(), D, D, 1, code, kw.data_ptr(), _hip.stream(W.device))
    return kw


def head_mixer(x: torch.Tensor, kweight: torch.Tensor, beta: torch.Tensor, out: torch.Tensor = None) -> torch.Tensor:
    """HadamardHeadMixerFused.forward (fht_cuda.py:650-662) on x [B, 32, T, D]
    (any strides with a unit inner one); returns the token-major [B, T, 32*D]
    rows (the layout after transpose(1, 2)), written into ``out`` if given (a
    [B, T, 32*D] view with unit inner stride and stride(0) == T*stride(1),
    e.g. one head group's columns of a [B, T, n_embd] tensor)."""
    _hip.require_device(x, "input")
    B, Hh, T, D = x.shape
    assert Hh == 32, f"the head mixer takes 32 heads, got {Hh}"
    dt = x.dtype
    if x.stride(3) != 1:
        x = x.contiguous()
    if out is None:
        y = torch.empty(B, T, 32 * D, device=x.device, dtype=dt)
    else:
        y = out
        assert tuple(y.shape) == (B, T, 32 * D) and y.dtype == dt and y.stride(2) == 1, "head mixer output view"
        assert B == 1 or y.stride(0) == T * y.stride(1), "head mixer output rows must be evenly spaced"
    if B * T == 0:
        return y
    if half_scales_used(dt, D, D):
        check_half_range("head mixer beta", beta)
    b = beta.detach().float().contiguous()
    esz = x.element_size()
    nbytes = 2 * B * T * 32 * D * esz + kweight.numel() + 4 * D
    flops = B * T * (2 * 32 * D * D + 10 * 32 * D + 32 * D)
    _hip.call("walsh_head_mixer_fwd", x.data_ptr(), B, T, D, x.stride(0), x.stride(1), x.stride(2),
              kweight.data_ptr(), b.data_ptr(), y.data_ptr(), y.stride(1), _hip.dtype_code(dt), _hip.stream(x.device),
              kernel="head_mixer<%s>" % ("bf16" if dt == torch.bfloat16 else "f32"), nbytes=nbytes, flops=flops)
    return y


def head_mixer_proj_supported(x: torch.Tensor, rows: int) -> bool:
    """Can head_mixer_proj take x [B, 32, T, 16] (bf16, 4-element aligned
    strides and pointer) at this many rows?  Above PAIR_MAX_TILES_ROWS tiles
    the output projection's whole-row kernel is the faster second launch."""
    return (x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 4 and tuple(x.shape[1:2]) == (32,)
            and x.shape[3] == 16 and x.stride(3) == 1 and all(st % 4 == 0 for st in x.stride()[:3])
            and x.data_ptr() % 8 == 0 and 0 < rows <= 16 * PAIR_MAX_TILES_ROWS)


def head_mixer_proj(x: torch.Tensor, mix_kweight: torch.Tensor, mix_beta: torch.Tensor, proj_kweight: torch.Tensor,
                    proj_alpha: torch.Tensor, proj_beta: torch.Tensor) -> torch.Tensor:
    """The head mixer (HadamardHeadMixerFused.forward, fht_cuda.py:650-662) and
    the attention output projection (a 16x16 HadamardLinear, fht_cuda.py:489-519)
    on x [B, 32, T, 16] bf16 in one launch: the token-major rows [B, T, 512],
    bitwise head_mixer followed by hadamard_linear."""
    _hip.require_device(x, "input")
    B, Hh, T, D = x.shape
    assert Hh == 32 and D == 16 and x.dtype == torch.bfloat16, f"head_mixer_proj: x {tuple(x.shape)} {x.dtype}"
    y = torch.empty(B, T, 512, device=x.device, dtype=x.dtype)
    if B * T == 0:
        return y
    mb = mix_beta.detach().float().contiguous()
    pa = proj_alpha.detach().float().contiguous()
    pb = proj_beta.detach().float().contiguous()
    assert mb.numel() == 16 and pa.numel() == 512 and pb.numel() == 512, "head_mixer_proj: parameter shapes"
    rows = B * T
    nbytes = 2 * rows * 512 * 2 + mix_kweight.numel() + proj_kweight.numel() + 4 * (16 + 1024)
    flops = rows * 2 * (2 * 32 * 16 * 16 + 10 * 32 * 16 + 32 * 16)
    _hip.call("walsh_head_mixer_proj_fwd", x.data_ptr(), B, T, x.stride(0), x.stride(1), x.stride(2),
              mix_kweight.data_ptr(), mb.data_ptr(), proj_kweight.data_ptr(), pa.data_ptr(), pb.data_ptr(),
              y.data_ptr(), 512, _hip.dtype_code(x.dtype), _hip.stream(x.device),
              kernel="head_mixer_proj<bf16>", nbytes=nbytes, flops=flops)
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
    (physics.py:66-82); B from octonion_prepare in x.dtype; beta None = ones."""
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
    beta_p = 0 if beta is None else beta.detach().float().contiguous().data_ptr()
    esz = x.element_size()
    nbytes = rows * 8 * (in_o + out_o) * esz + 8 * out_o * ((in_o + 3) // 4) + 4 * out_o
    flops = 2 * rows * (8 * in_o) * (8 * out_o)
    _hip.call("walsh_octonion_linear_fwd", xv.data_ptr(), ldx, rows, in_o, out_o, B.data_ptr(), beta_p,
              y.data_ptr(), 8 * out_o, _hip.dtype_code(x.dtype), _hip.stream(x.device),
              kernel="octonion_gemm_kernel<%s>" % ("bf16" if x.dtype == torch.bfloat16 else "f32"),
              nbytes=nbytes, flops=flops)
    return y


def octonion_fused_linear(x: torch.Tensor, in_o: int, out_o: int, B: torch.Tensor,
                          beta: torch.Tensor) -> torch.Tensor:
    """The reference GPU module's forward (OctonionFusedLinear.forward,
    cayley_dickson_cuda.py:650-668): x rounded to bf16, the bf16 product with
    float32 accumulation rounded to bf16, times the float32 beta -> float32
    [..., 8*out_o].  B from octonion_prepare in bf16; beta None = ones."""
    _hip.require_device(x, "input")
    assert B.dtype == torch.bfloat16, "the fused layer multiplies bf16 operands"
    K = 8 * in_o
    lead = x.shape[:-1]
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    xv, rows, ldx = _rows_view(x, K)
    y = torch.empty(lead + (8 * out_o,), device=x.device, dtype=torch.float32)
    if rows == 0:
        return y
    if ldx % 8 or xv.data_ptr() % 16:
        xv = xv.reshape(rows, -1)[:, :K].contiguous()
        ldx = K
    beta_p = 0 if beta is None else beta.detach().float().contiguous().data_ptr()
    nbytes = rows * 8 * (2 * in_o + 4 * out_o) + 8 * out_o * ((in_o + 3) // 4) + 4 * out_o
    flops = 2 * rows * (8 * in_o) * (8 * out_o)
    _hip.call("walsh_octonion_fused_fwd", xv.data_ptr(), ldx, rows, in_o, out_o, B.data_ptr(), beta_p,
              y.data_ptr(), 8 * out_o, _hip.stream(x.device),
              kernel="octonion_fused<bf16,f32>", nbytes=nbytes, flops=flops)
    return y


def octonion_prepare_t(packed: torch.Tensor, in_o: int, out_o: int, beta: torch.Tensor,
                       dtype: torch.dtype) -> torch.Tensor:
    """Transposed block matrix with beta folded in, [8*in_o, roundup(8*out_o, 32)]:
    the weights of the input-gradient GEMM."""
    _hip.require_device(packed, "packed weight")
    assert tuple(packed.shape) == (8, out_o, (in_o + 3) // 4), f"packed shape {tuple(packed.shape)}"
    Np = (8 * out_o + 31) // 32 * 32
    Bt = torch.empty(8 * in_o * Np, device=packed.device, dtype=dtype)
    beta = beta.detach().float().contiguous()
    _hip.call("walsh_octonion_prepare_t", packed.contiguous().data_ptr(), in_o, out_o, beta.data_ptr(),
              Bt.data_ptr(), _hip.dtype_code(dtype), _hip.stream(packed.device))
    return Bt


def octonion_linear_bwd(x: torch.Tensor, gy: torch.Tensor, in_o: int, out_o: int, packed: torch.Tensor,
                        beta: torch.Tensor, latent: torch.Tensor = None, need=(True, True, True)):
    """Backward of octonion_linear (CayleyDicksonFunction.backward,
    cayley_dickson_cuda.py:500-567, with the STE of physics.py:48-50).

    Returns (gx, dweight, dbeta); entries not requested in ``need`` are None.
    gx = (gy .* beta) B on the HIP GEMM (transposed block matrix); the
    parameter gradients come from C = gy^T x ([8*out_o, 8*in_o], K = tokens:
    transposed operands, split-K GEMM with float32 partial sums, then the
    fold) in walsh_octonion_bwd_params."""
    _hip.require_device(x, "input")
    dt = x.dtype
    assert gy.dtype == dt, f"gradient dtype {gy.dtype} != input dtype {dt}"
    xr = x.reshape(-1, 8 * in_o)
    gr = gy.reshape(-1, 8 * out_o)
    want_x, want_w, want_b = need
    gx = dw = db = None
    if want_x:
        Bt = octonion_prepare_t(packed, in_o, out_o, beta, dt)
        gx = octonion_linear(gr, out_o, in_o, Bt, None).view(x.shape)
    if want_w or want_b:
        dw = torch.empty(8, out_o, in_o, device=x.device, dtype=torch.float32) if want_w else None
        db = torch.empty(out_o, device=x.device, dtype=torch.float32) if want_b else None
        lat = latent.detach().float().contiguous() if (latent is not None and want_w) else None
        beta = beta.detach().float().contiguous()
        ptr = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
        M = gr.shape[0]
        if M == 0:
            C = torch.zeros(8 * out_o, 8 * in_o, device=x.device, dtype=torch.float32)
            _hip.call("walsh_octonion_bwd_fold", C.data_ptr(), 8 * in_o, 1, 0, packed.contiguous().data_ptr(), in_o,
                      out_o, beta.data_ptr(), ptr(lat), ptr(dw), ptr(db), _hip.stream(x.device))
        else:
            gr, xr = gr.contiguous(), xr.contiguous()
            nws = _hip.lib().walsh_octonion_bwd_params_workspace_bytes(M, in_o, out_o, _hip.dtype_code(dt))
            ws = torch.empty(nws, device=x.device, dtype=torch.uint8)
            esz = x.element_size()
            _hip.call("walsh_octonion_bwd_params", gr.data_ptr(), gr.stride(0), xr.data_ptr(), xr.stride(0), M, in_o,
                      out_o, packed.contiguous().data_ptr(), beta.data_ptr(), ptr(lat), ptr(dw), ptr(db),
                      _hip.dtype_code(dt), ws.data_ptr(), nws, _hip.stream(x.device),
                      kernel="octonion_bwd_params<%s>" % ("bf16" if dt == torch.bfloat16 else "f32"),
                      nbytes=2 * M * 8 * (in_o + out_o) * esz, flops=2 * M * 64 * in_o * out_o)
    return gx, dw, db


# ------------------------------------------------------------------ decode attention

DECODE_HEAD_DIMS = (16, 32, 64, 128)


def decode_attention_supported(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    """q [B, H, 1, D]; k, v [B, H, L, D] views with unit inner stride."""
    if not (q.is_cuda and q.dim() == 4 and q.shape[2] == 1 and q.shape[-1] in DECODE_HEAD_DIMS):
        return False
    if q.dtype not in (torch.float32, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        return False
    if k.stride() != v.stride() or k.stride(-1) != 1 or q.stride(-1) != 1 or k.shape != v.shape:
        return False
    ok = all(st % 8 == 0 for st in (q.stride(0), q.stride(1), k.stride(0), k.stride(1), k.stride(2)))
    return ok and all(t.data_ptr() % 16 == 0 for t in (q, k, v))


def decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float = None) -> torch.Tensor:
    """softmax(q k^T * scale) v for one query per (sequence, head) over the
    L cached positions (no mask): q [B, H, 1, D], k / v [B, H, L, D] (the KV
    cache's head-major storage, read in place) -> [B, H, 1, D] in q.dtype."""
    _hip.require_device(q, "query")
    B, H, _, D = q.shape
    L = k.shape[2]
    scale = 1.0 / (D ** 0.5) if scale is None else scale
    o = torch.empty(B, H, 1, D, device=q.device, dtype=q.dtype)
    nws = _hip.lib().walsh_decode_attention_workspace_bytes(B, H, L, D)
    ws = torch.empty(max(nws, 4) // 4, device=q.device, dtype=torch.float32)
    esz = q.element_size()
    _hip.call("walsh_decode_attention", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(),
              k.stride(0), k.stride(1), k.stride(2), B, H, L, D, float(scale), o.data_ptr(), o.stride(0), o.stride(1),
              _hip.dtype_code(q.dtype), ws.data_ptr(), nws, _hip.stream(q.device),
              kernel="decode_attn_partial_kernel<%s,%d>" % ("bf16" if q.dtype == torch.bfloat16 else "f32", D),
              nbytes=2 * B * H * L * D * esz + 2 * B * H * D * esz, flops=4 * B * H * L * D)
    return o


def decode_attention_static(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                            scale: float = None) -> torch.Tensor:
    """decode_attention through walsh_decode_attention_static: the split-K
    partials stay in the library's fixed per-GPU scratch array, so the call
    allocates nothing (``out`` [B, H, 1, D] in q.dtype is the caller's).
    Calls that overlap on one GPU race on that array; shapes whose partials
    exceed it raise WalshHipError."""
    _hip.require_device(q, "query")
    B, H, _, D = q.shape
    L = k.shape[2]
    assert tuple(out.shape) == (B, H, 1, D) and out.dtype == q.dtype and out.stride(-1) == 1, "output view"
    scale = 1.0 / (D ** 0.5) if scale is None else scale
    esz = q.element_size()
    _hip.call("walsh_decode_attention_static", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(),
              k.stride(0), k.stride(1), k.stride(2), B, H, L, D, float(scale), out.data_ptr(), out.stride(0),
              out.stride(1), _hip.dtype_code(q.dtype), _hip.stream(q.device),
              kernel="decode_attn_partial_kernel<%s,%d>" % ("bf16" if q.dtype == torch.bfloat16 else "f32", D),
              nbytes=2 * B * H * L * D * esz + 2 * B * H * D * esz, flops=4 * B * H * L * D)
    return out


PREFILL_HEAD_DIMS = (16, 32, 64, 128)


def prefill_attention_supported(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    """q, k, v [B, H, T, D] views (same T) with unit inner stride, bf16."""
    if not (q.is_cuda and q.dim() == 4 and q.shape[-1] in PREFILL_HEAD_DIMS and q.dtype == torch.bfloat16):
        return False
    if k.dtype != q.dtype or v.dtype != q.dtype or k.shape != q.shape or v.shape != q.shape:
        return False
    if k.stride() != v.stride() or any(t.stride(-1) != 1 for t in (q, k, v)):
        return False
    ok = all(st % 8 == 0 and st >= 0 for t in (q, k) for st in t.stride()[:3])
    return ok and all(t.data_ptr() % 16 == 0 for t in (q, k, v))


def prefill_attention_preferred(q: torch.Tensor) -> bool:
    """Whether the model should route causal prefill attention here rather
    than to SDPA: head_dim 16, where the whole-head kernel is VALU-bound
    and measured 2.4x faster than SDPA at T = 1024 (51 vs 125 us per layer,
    config 2), and head_dim 128 (the 128-query matrix-core kernel: 1.18 ms
    against SDPA's 2.33 ms per layer at config 5).  Head dims 32 and 64 stay
    on SDPA."""
    return q.shape[-1] in (16, 128)


def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float = None) -> torch.Tensor:
    """softmax(q k^T * scale + causal mask) v (SDPA with is_causal=True) for
    q, k, v [B, H, T, D] views (e.g. the transposed [B, T, H, D] projections)
    -> contiguous [B, H, T, D]."""
    _hip.require_device(q, "query")
    B, H, T, D = q.shape
    scale = 1.0 / (D ** 0.5) if scale is None else scale
    o = torch.empty(B, H, T, D, device=q.device, dtype=q.dtype)
    qs, ks = q.stride(), k.stride()
    _hip.call("walsh_prefill_attention", q.data_ptr(), qs[0], qs[1], qs[2], k.data_ptr(), v.data_ptr(), ks[0], ks[1],
              ks[2], B, H, T, D, float(scale), o.data_ptr(), H * T * D, T * D, D, _hip.dtype_code(q.dtype),
              _hip.stream(q.device), kernel="prefill_attn_kernel<bf16,%d>" % D,
              nbytes=4 * B * H * T * D * q.element_size(), flops=2 * B * H * T * T * D)
    return o


# ------------------------------------------------------------------ channel modulation

def _groups(x: torch.Tensor) -> torch.Tensor:
    """[G, T, C] with unit column stride, 4-aligned row stride and the groups
    laid out one after another (what the channel-modulation kernels read)."""
    assert x.dim() == 3, "channel modulation takes [groups, T, C]"
    G, T, C = x.shape
    ok = x.stride(-1) == 1 and x.stride(1) % 4 == 0 and x.stride(1) >= C and x.stride(0) == T * x.stride(1)
    ok = ok and x.data_ptr() % (8 if x.dtype == torch.bfloat16 else 16) == 0
    return x if ok else x.contiguous()


def chanmod_fwd(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, scale_temp: torch.Tensor, n_blocks: int,
                residual_scale: float, shift_scale: float = 0.1, norm_w: torch.Tensor = None, eps: float = 1e-6,
                add_input: bool = False):
    """HadamardChannelModulation.forward (moe.py:676-727) on x [G, T, C]
    (float32 or bfloat16), with the context MLP weights w1 [hidden, C] and
    w2 [2*n_blocks, hidden] as float32 values (ternary code*gamma, or the
    latent weights).  With ``norm_w`` the input is RMSNorm(x)*norm_w first;
    with ``add_input`` x is added to the result (the block's residual,
    mhc.py:531).  Returns (y [G, T, C] in x.dtype, scale_shift float32
    [G, 2*n_blocks] = scale then shift per group)."""
    _hip.require_device(x, "input")
    x = _groups(x)
    G, T, C = x.shape
    dev = x.device
    w1f = w1.detach().float().contiguous()
    w2f = w2.detach().float().contiguous()
    hidden = w1f.shape[0]
    assert w1f.shape == (hidden, C) and w2f.shape == (2 * n_blocks, hidden), "context MLP shapes"
    st = scale_temp.detach().float().reshape(-1)[:1].contiguous()
    nw = None if norm_w is None else norm_w.detach().float().contiguous()
    y = torch.empty(G, T, C, device=dev, dtype=x.dtype)
    ss = torch.empty(G, 2 * n_blocks, device=dev, dtype=torch.float32)
    nws = _hip.lib().walsh_chanmod_workspace_bytes(G, T, C)
    ws = torch.empty(max(nws, 4) // 4, device=dev, dtype=torch.float32)
    esz = x.element_size()
    _hip.call("walsh_chanmod_fwd", x.data_ptr(), x.stride(1), G, T, C, _hip.ptr(nw), float(eps), w1f.data_ptr(),
              hidden, w2f.data_ptr(), int(n_blocks), st.data_ptr(), float(residual_scale), float(shift_scale),
              int(bool(add_input)), y.data_ptr(), C, ss.data_ptr(), _hip.dtype_code(x.dtype), ws.data_ptr(), nws,
              _hip.stream(dev), kernel="chanmod<%s>" % ("bf16" if x.dtype == torch.bfloat16 else "f32"),
              nbytes=2 * G * T * C * esz, flops=0)
    return y, ss


def chanmod_apply(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, residual_scale: float,
                  shift_scale: float = 0.1) -> torch.Tensor:
    """ChannelModFunction's forward (moe.py:116-153): x [G, T, C], scale /
    shift [G, n_blocks] -> x + r*(x*scale + shift_scale*shift - x) per block."""
    _hip.require_device(x, "input")
    x = _groups(x)
    G, T, C = x.shape
    sc = scale.detach().float().contiguous()
    sh = shift.detach().float().contiguous()
    nb = sc.shape[-1]
    assert sc.shape == (G, nb) and sh.shape == (G, nb), "scale / shift must be [groups, n_blocks]"
    y = torch.empty(G, T, C, device=x.device, dtype=x.dtype)
    _hip.call("walsh_chanmod_apply", x.data_ptr(), x.stride(1), G, T, C, nb, sc.data_ptr(), sh.data_ptr(), nb,
              float(residual_scale), float(shift_scale), y.data_ptr(), C, _hip.dtype_code(x.dtype),
              _hip.stream(x.device))
    return y


def chanmod_bwd(gy: torch.Tensor, x: torch.Tensor, scale: torch.Tensor, residual_scale: float,
                shift_scale: float = 0.1):
    """ChannelModFunction's backward (moe.py:155-199, :235-256): returns
    (gx in x.dtype, dscale, dshift float32 [G, n_blocks])."""
    _hip.require_device(x, "input")
    x = _groups(x)
    G, T, C = x.shape
    g = _groups(gy.to(x.dtype))
    assert g.shape == x.shape, "gradient shape"
    sc = scale.detach().float().contiguous()
    nb = sc.shape[-1]
    gx = torch.empty(G, T, C, device=x.device, dtype=x.dtype)
    ds = torch.empty(G, nb, device=x.device, dtype=torch.float32)
    dh = torch.empty(G, nb, device=x.device, dtype=torch.float32)
    nws = _hip.lib().walsh_chanmod_workspace_bytes(G, T, C)
    ws = torch.empty(max(nws, 4) // 4, device=x.device, dtype=torch.float32)
    _hip.call("walsh_chanmod_bwd", g.data_ptr(), g.stride(1), x.data_ptr(), x.stride(1), G, T, C, nb, sc.data_ptr(),
              nb, float(residual_scale), float(shift_scale), gx.data_ptr(), C, ds.data_ptr(), dh.data_ptr(),
              _hip.dtype_code(x.dtype), ws.data_ptr(), nws, _hip.stream(x.device))
    return gx, ds, dh


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


def sinkhorn_bwd(h: torch.Tensor, g: torch.Tensor, n_iter: int = 20, eps: float = 1e-8) -> torch.Tensor:
    """Gradient of ``sinkhorn`` wrt h for the output gradient g (float32, h's shape)."""
    _hip.require_device(h, "H")
    n = h.shape[-1]
    hf = h.detach().float().contiguous()
    gf = g.float().contiguous()
    assert gf.shape == hf.shape, "gradient shape"
    dh = torch.empty_like(hf)
    batch = hf.numel() // (n * n)
    _hip.call("walsh_sinkhorn_bwd", hf.data_ptr(), gf.data_ptr(), batch, n, int(n_iter), float(eps), dh.data_ptr(),
              _hip.stream(h.device))
    return dh


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


def mhc_post_pre_supported(n: int, C: int, dtype: torch.dtype) -> bool:
    """Shapes walsh_mhc_post_pre_norm_fwd takes (the LDS tile of
    walsh_mhc_pre_norm_fwd, stream rows of whole 16-byte chunks)."""
    esz = 2 if dtype == torch.bfloat16 else 4
    return mhc_pre_supported(n, C, dtype) and (n * C) % 16 == 0 and (C * esz) % 16 == 0


def mhc_post_pre_norm(x_old: torch.Tensor, out: torch.Tensor, h_res_prev: torch.Tensor, h_post_prev: torch.Tensor,
                      phi_frag: torch.Tensor, coef: torch.Tensor, bias_cat: torch.Tensor, rms_eps: float,
                      norm_w: torch.Tensor = None, norm_eps: float = 1e-6, n_iter: int = 20, sk_eps: float = 1e-8):
    """mhc_post of the previous stream fused with mhc_pre_norm of the next:
    x_new = H_res_prev @ x_old + H_post_prev^T (x) out is formed as the
    mapping kernel loads its tile (mhc.py:366-381 then :283-318, :345-364).
    Returns (x_new, layer_in, h_pre, h_post, h_res); x_new is bitwise
    mhc_post's result."""
    _hip.require_device(x_old, "stream input")
    n, C = x_old.shape[-2], x_old.shape[-1]
    lead = x_old.shape[:-2]
    xo = x_old if x_old.is_contiguous() else x_old.contiguous()
    M = xo.numel() // (n * C)
    dev = x_old.device
    o = out.to(x_old.dtype)
    o = o if o.is_contiguous() else o.contiguous()
    assert o.numel() == M * C, "layer output shape"
    hr = h_res_prev.detach().float().contiguous()
    hp = h_post_prev.detach().float().contiguous()
    x_new = torch.empty_like(xo)
    layer_in = torch.empty(lead + (C,), device=dev, dtype=x_old.dtype)
    h_pre = torch.empty(lead + (n,), device=dev, dtype=torch.float32)
    h_post = torch.empty(lead + (n,), device=dev, dtype=torch.float32)
    h_res = torch.empty(lead + (n, n), device=dev, dtype=torch.float32)
    if M == 0:
        return x_new, layer_in, h_pre, h_post, h_res
    assert phi_frag.dtype == x_old.dtype and phi_frag.numel() == 32 * n * C, "phi_frag layout"
    nw = None
    if norm_w is not None:
        nw = norm_w.detach().float().contiguous()
        assert nw.numel() == C
    esz = x_old.element_size()
    nbytes = M * (2 * n * C + 2 * C) * esz + M * (3 * n + 2 * n * n) * 4 + 32 * n * C * esz
    flops = M * (2 * n * C * 32 + 2 * n * C + 2 * n * C + n * C * (2 * n + 2))
    _hip.call("walsh_mhc_post_pre_norm_fwd", xo.data_ptr(), n * C, o.data_ptr(), C, hr.data_ptr(), hp.data_ptr(),
              x_new.data_ptr(), n * C, M, n, C, phi_frag.data_ptr(), coef.data_ptr(), bias_cat.data_ptr(),
              float(rms_eps), int(n_iter), float(sk_eps), h_pre.data_ptr(), h_post.data_ptr(), h_res.data_ptr(),
              layer_in.data_ptr(), C, _hip.ptr(nw), float(norm_eps), _hip.dtype_code(x_old.dtype), _hip.stream(dev),
              kernel="mhc_post_pre2_kernel<%s>" % ("bf16" if x_old.dtype == torch.bfloat16 else "f32"),
              nbytes=nbytes, flops=flops)
    return x_new, layer_in, h_pre, h_post, h_res


def phi_fragments32(phi_cat: torch.Tensor) -> torch.Tensor:
    """phi_cat [32, K] -> 16x16x32 matrix-core fragment order [K/32][2][64][8]
    (lane = 16*kq + n holds phi[16*tile + n][32*ks + 8*kq .. +7])."""
    K = phi_cat.shape[1]
    return phi_cat.view(2, 16, K // 32, 4, 8).permute(2, 0, 3, 1, 4).contiguous()


def mhc_pre_wide_supported(n: int, C: int) -> bool:
    """Whether walsh_mhc_pre_wide_fwd handles this shape (rows too long for
    the LDS-tile kernel, up to n_embd 4096)."""
    return n <= 4 and (n * C) % 32 == 0 and C % 4 == 0 and C <= 4096


def mhc_pre_wide(x: torch.Tensor, phi_frag32: torch.Tensor, coef: torch.Tensor, bias_cat: torch.Tensor,
                 rms_eps: float, norm_w: torch.Tensor = None, norm_eps: float = 1e-6, n_iter: int = 20,
                 sk_eps: float = 1e-8):
    """mhc_pre_norm for long rows: split-K projection, then per-token
    constraints and layer input (two launches; workspace from the caching
    allocator)."""
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
    assert phi_frag32.dtype == x.dtype and phi_frag32.numel() == 32 * n * C, "phi_frag32 layout"
    nw = None
    if norm_w is not None:
        nw = norm_w.detach().float().contiguous()
        assert nw.numel() == C
    wsb = _hip.lib().walsh_mhc_pre_wide_workspace(M, n, C)
    ws = torch.empty(max(wsb, 4), device=dev, dtype=torch.uint8)
    esz = x.element_size()
    # algorithmic bytes: the stream rows read once (the projection and the
    # apply launch each read them; the second read is measured traffic, not
    # algorithmic), the layer input and the mappings written once, phi once
    nbytes = M * n * C * esz + M * C * esz + M * (2 * n + n * n) * 4 + 32 * n * C * esz
    flops = M * (2 * n * C * 32 + 2 * n * C + 2 * n * C)
    _hip.call("walsh_mhc_pre_wide_fwd", xv.data_ptr(), n * C, M, n, C, phi_frag32.data_ptr(), coef.data_ptr(),
              bias_cat.data_ptr(), float(rms_eps), int(n_iter), float(sk_eps), h_pre.data_ptr(), h_post.data_ptr(),
              h_res.data_ptr(), layer_in.data_ptr(), C, _hip.ptr(nw), float(norm_eps), ws.data_ptr(), ws.numel(),
              _hip.dtype_code(x.dtype), _hip.stream(dev),
              kernel="mhc_proj+apply<%s>" % ("bf16" if x.dtype == torch.bfloat16 else "f32"), nbytes=nbytes,
              flops=flops)
    return layer_in, h_pre, h_post, h_res


def mhc_post_pre_wide_supported(n: int, C: int, dtype: torch.dtype) -> bool:
    """Whether walsh_mhc_post_pre_wide_fwd handles this shape (bf16, C a
    multiple of 32 up to 4096)."""
    return dtype == torch.bfloat16 and n <= 4 and C % 32 == 0 and C <= 4096


def mhc_post_pre_wide(x_old: torch.Tensor, out: torch.Tensor, h_res_prev: torch.Tensor, h_post_prev: torch.Tensor,
                      phi_frag32: torch.Tensor, coef: torch.Tensor, bias_cat: torch.Tensor, rms_eps: float,
                      norm_w: torch.Tensor = None, norm_eps: float = 1e-6, n_iter: int = 20, sk_eps: float = 1e-8):
    """mhc_post of the previous stream fused with mhc_pre_wide of the next
    (mhc.py:366-381 then :283-364): the projection launch forms x_new while
    it loads x_old and out, stores it and feeds it to the matrix cores; the
    per-token launch reads x_new.  Returns (x_new, layer_in, h_pre, h_post,
    h_res); x_new is bitwise mhc_post's result."""
    _hip.require_device(x_old, "stream input")
    n, C = x_old.shape[-2], x_old.shape[-1]
    lead = x_old.shape[:-2]
    xo = x_old if x_old.is_contiguous() else x_old.contiguous()
    M = xo.numel() // (n * C)
    dev = x_old.device
    o = out.to(x_old.dtype)
    o = o if o.is_contiguous() else o.contiguous()
    assert o.numel() == M * C, "layer output shape"
    hr = h_res_prev.detach().float().contiguous()
    hp = h_post_prev.detach().float().contiguous()
    x_new = torch.empty_like(xo)
    layer_in = torch.empty(lead + (C,), device=dev, dtype=x_old.dtype)
    h_pre = torch.empty(lead + (n,), device=dev, dtype=torch.float32)
    h_post = torch.empty(lead + (n,), device=dev, dtype=torch.float32)
    h_res = torch.empty(lead + (n, n), device=dev, dtype=torch.float32)
    if M == 0:
        return x_new, layer_in, h_pre, h_post, h_res
    assert phi_frag32.dtype == x_old.dtype and phi_frag32.numel() == 32 * n * C, "phi_frag32 layout"
    nw = None
    if norm_w is not None:
        nw = norm_w.detach().float().contiguous()
        assert nw.numel() == C
    wsb = _hip.lib().walsh_mhc_pre_wide_workspace(M, n, C)
    ws = torch.empty(max(wsb, 4), device=dev, dtype=torch.uint8)
    esz = x_old.element_size()
    # algorithmic bytes: x_old and out read once, x_new written once, the
    # layer input and the mappings written once, phi once (the per-token
    # launch's read of x_new is measured traffic, not algorithmic)
    nbytes = M * (2 * n * C + 2 * C) * esz + M * (3 * n + 2 * n * n) * 4 + 32 * n * C * esz
    flops = M * (2 * n * C * 32 + 2 * n * C + 2 * n * C + n * C * (2 * n + 2))
    _hip.call("walsh_mhc_post_pre_wide_fwd", xo.data_ptr(), n * C, o.data_ptr(), C, hr.data_ptr(), hp.data_ptr(),
              x_new.data_ptr(), n * C, M, n, C, phi_frag32.data_ptr(), coef.data_ptr(), bias_cat.data_ptr(),
              float(rms_eps), int(n_iter), float(sk_eps), h_pre.data_ptr(), h_post.data_ptr(), h_res.data_ptr(),
              layer_in.data_ptr(), C, _hip.ptr(nw), float(norm_eps), ws.data_ptr(), ws.numel(),
              _hip.dtype_code(x_old.dtype), _hip.stream(dev), kernel="mhc_post_proj+apply<bf16>", nbytes=nbytes,
              flops=flops)
    return x_new, layer_in, h_pre, h_post, h_res


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


def _dense(t: torch.Tensor, dtype=None) -> torch.Tensor:
    t = t if dtype is None else t.to(dtype)
    return t if t.is_contiguous() else t.contiguous()


def _check_extents(fn: str, M: int, operands) -> None:
    """Host-side bounds check for the raw-pointer stream-mixing kernels: each
    (tensor, elements per token) must hold exactly M tokens' worth."""
    for i, (t, per) in enumerate(operands):
        if t.numel() != M * per:
            raise ValueError(f"{fn}: operand {i} has {t.numel()} elements, the kernel addresses {M} x {per}")


def mhc_aggregate(x: torch.Tensor, h_pre: torch.Tensor) -> torch.Tensor:
    """layer_in = H_pre @ x (mhc.py:366) for x [..., n, C], h_pre [..., 1, n] or
    [..., n]; float32 sums, result in x.dtype [..., C]."""
    _hip.require_device(x, "stream input")
    n, C = x.shape[-2], x.shape[-1]
    xv = _dense(x)
    M = xv.numel() // (n * C)
    hp = _dense(h_pre.detach(), torch.float32)
    assert hp.numel() == M * n, "h_pre shape"
    li = torch.empty(x.shape[:-2] + (C,), device=x.device, dtype=x.dtype)
    _hip.call("walsh_mhc_aggregate_fwd", xv.data_ptr(), hp.data_ptr(), li.data_ptr(), M, n, C,
              _hip.dtype_code(x.dtype), _hip.stream(x.device))
    return li


def mhc_aggregate_bwd(x: torch.Tensor, h_pre: torch.Tensor, d_li: torch.Tensor):
    """(dx [..., n, C] in x.dtype, dh_pre float32 h_pre's shape) of mhc_aggregate."""
    n, C = x.shape[-2], x.shape[-1]
    xv = _dense(x)
    M = xv.numel() // (n * C)
    hp = _dense(h_pre.detach(), torch.float32)
    g = _dense(d_li, x.dtype)
    # the kernel walks dense [M][n][C] / [M][C] / [M][n] rows with raw
    # pointers: every operand must hold exactly that many elements
    _check_extents("mhc_aggregate_bwd", M, ((xv, n * C), (hp, n), (g, C)))
    dx = torch.empty_like(xv)
    dh = torch.empty(hp.shape, device=x.device, dtype=torch.float32)
    _hip.call("walsh_mhc_aggregate_bwd", xv.data_ptr(), hp.data_ptr(), g.data_ptr(), dx.data_ptr(), dh.data_ptr(),
              M, n, C, _hip.dtype_code(x.dtype), _hip.stream(x.device))
    return dx, dh


def mhc_post_bwd(x: torch.Tensor, out: torch.Tensor, h_res: torch.Tensor, h_post: torch.Tensor,
                 d_new: torch.Tensor):
    """Gradients (dx, d_out, dh_res, dh_post) of mhc_post; dx / d_out in
    x.dtype, the mappings' gradients float32 in their input shapes."""
    n, C = x.shape[-2], x.shape[-1]
    xv = _dense(x)
    M = xv.numel() // (n * C)
    o = _dense(out, x.dtype)
    hr = _dense(h_res.detach(), torch.float32)
    hq = _dense(h_post.detach(), torch.float32)
    g = _dense(d_new, x.dtype)
    _check_extents("mhc_post_bwd", M, ((xv, n * C), (o, C), (hr, n * n), (hq, n), (g, n * C)))
    dx = torch.empty_like(xv)
    dout = torch.empty_like(o)
    dhr = torch.empty(hr.shape, device=x.device, dtype=torch.float32)
    dhq = torch.empty(hq.shape, device=x.device, dtype=torch.float32)
    esz = x.element_size()
    _hip.call("walsh_mhc_post_bwd", xv.data_ptr(), o.data_ptr(), hr.data_ptr(), hq.data_ptr(), g.data_ptr(),
              dx.data_ptr(), dout.data_ptr(), dhr.data_ptr(), dhq.data_ptr(), M, n, C, _hip.dtype_code(x.dtype),
              _hip.stream(x.device), kernel="mhc_post_bwd_kernel<%s>" % ("bf16" if x.dtype == torch.bfloat16 else "f32"),
              nbytes=M * (3 * n * C + 2 * C) * esz + M * (n * n + n) * 8, flops=M * n * C * (4 * n + 4))
    return dx, dout, dhr, dhq


# ------------------------------------------------------------------ MoE

def moe_router_fragments(w1: torch.Tensor, w2: torch.Tensor, dtype: torch.dtype):
    """Router weights W1 [H1, C], W2 [E, H1] in the fragment order of
    walsh_moe_route_fwd, as ``dtype`` elements: W1 -> [H1/16][C/16][64][4],
    W2 -> [ceil(E/16)][H1/16][64][4] with rows >= E zero (lane = 16*kq + m)."""
    H1, C = w1.shape
    E = w2.shape[0]
    assert C % 16 == 0 and H1 % 16 == 0, "router needs n_embd % 64 == 0"
    assert w2.shape[1] == H1, "router W2 shape"
    f1 = w1.detach().to(dtype).reshape(H1 // 16, 16, C // 16, 4, 4).permute(0, 2, 3, 1, 4).contiguous()
    ET = (E + 15) // 16
    w2p = torch.zeros(ET * 16, H1, device=w2.device, dtype=dtype)
    w2p[:E] = w2.detach().to(dtype)
    f2 = w2p.reshape(ET, 16, H1 // 16, 4, 4).permute(0, 2, 3, 1, 4).contiguous()
    return f1, f2


def moe_expert_fragments(gate_packed: torch.Tensor, up_packed: torch.Tensor, down_packed: torch.Tensor):
    """Packed expert codes (pack_ternary_weights layout: gate/up [E, H, 8],
    down [E, 32, H/4]) -> fragment order of walsh_moe_experts_fwd."""
    E, H, kb = gate_packed.shape
    assert kb == 8 and tuple(up_packed.shape) == (E, H, 8), "gate/up packed shape"
    assert tuple(down_packed.shape) == (E, 32, H // 4) and H % 16 == 0, "down packed shape"

    def gu(p):  # [e][nt][m][c][kq] -> [e][nt][c][kq][m]
        return p.reshape(E, H // 16, 16, 2, 4).permute(0, 1, 3, 4, 2).contiguous()

    down = down_packed.reshape(E, 2, 16, H // 16, 4).permute(0, 1, 3, 4, 2).contiguous()  # [e][mt][ks][kq][m]
    return gu(gate_packed), gu(up_packed), down


class MoERoute:
    """Device-side routing of one MoE call: topk_idx [M, k] int32, topk_w
    [M, k] float32, optional dense [M, E] outputs, and the per-expert token
    counts / probability sums, written by the kernels as [parts, E]
    per-workgroup partial sums.  ``count`` / ``probsum`` are the totals:
    set by moe_scatter, or summed from the partials on first access."""

    __slots__ = ("M", "E", "k", "topk_idx", "topk_w", "count_part", "probsum_part", "_count", "_probsum", "probs",
                 "mask", "weights")

    def __init__(self, M, E, k, dev, dense, parts):
        self.M, self.E, self.k = M, E, k
        self.topk_idx = torch.empty(M, k, device=dev, dtype=torch.int32)
        self.topk_w = torch.empty(M, k, device=dev, dtype=torch.float32)
        self.count_part = torch.empty(parts, E, device=dev, dtype=torch.int32)
        self.probsum_part = torch.empty(parts, E, device=dev, dtype=torch.float32)
        self._count = self._probsum = None
        if dense:
            d = torch.empty(3, M, E, device=dev, dtype=torch.float32)
            self.probs, self.mask, self.weights = d[0], d[1], d[2]
        else:
            self.probs = self.mask = self.weights = None

    @property
    def parts(self) -> int:
        return self.count_part.shape[0]

    @property
    def count(self):
        if self._count is None:
            self._count = self.count_part.sum(0, dtype=torch.int32)
        return self._count

    @property
    def probsum(self):
        if self._probsum is None:
            self._probsum = self.probsum_part.sum(0)
        return self._probsum


def _parts(M: int, per: int, dev) -> int:
    """Partial-sum rows of a routing launch: one per workgroup."""
    return max(1, min((M + per - 1) // per, 4 * _hip.cu_count(dev)))


def moe_route(x: torch.Tensor, w1f: torch.Tensor, w2f: torch.Tensor, H1: int, E: int, k: int, dense: bool = False,
              y: torch.Tensor = None) -> MoERoute:
    """Fused router (moe.py:418-447) on x [M, C] (unit inner stride): logits,
    softmax, top-k, renormalised weights, per-expert counts and probability
    sums.  If y [M, 32E] is given, the blocks of unselected experts are zeroed."""
    _hip.require_device(x, "input")
    dt = x.dtype
    assert w1f.dtype == dt and w2f.dtype == dt, "router fragments must be in the activation dtype"
    xv, M, ldx = _rows_view(x, x.shape[-1])
    C = x.shape[-1]
    r = MoERoute(M, E, k, x.device, dense, _parts(M, 64, x.device))
    ldy, ydt = 0, dt
    if y is not None:
        assert y.shape[-1] == 32 * E and y.stride(-1) == 1, "output layout"
        ldy, ydt = (y.stride(0) if y.dim() == 2 else 32 * E), y.dtype
    esz = x.element_size()
    nbytes = M * C * esz + (H1 * C + E * H1) * esz + M * k * 8
    if y is not None:
        nbytes += M * (E - k) * 32 * y.element_size()
    _hip.call("walsh_moe_route_fwd", xv.data_ptr(), ldx, M, C, H1, w1f.data_ptr(), w2f.data_ptr(), E, k,
              _hip.ptr(r.probs), _hip.ptr(r.mask), _hip.ptr(r.weights), r.topk_idx.data_ptr(), r.topk_w.data_ptr(),
              r.count_part.data_ptr(), r.probsum_part.data_ptr(), r.parts, _hip.ptr(y), ldy, _hip.dtype_code(dt),
              _hip.dtype_code(ydt), _hip.stream(x.device),
              kernel="moe_route_kernel<%s>" % ("bf16" if dt == torch.bfloat16 else "f32"), nbytes=nbytes,
              flops=2 * M * (C * H1 + H1 * E))
    return r


def moe_router_wide_supported(x2d: torch.Tensor, H: int, E: int, k: int) -> bool:
    """Whether walsh_moe_router_wide_fwd takes this bf16 router: C % 256 == 0,
    H % 128 == 0, H <= 1024, E <= 128 with E % 4 == 0, k <= 8, 16-byte aligned rows, x under
    2^31 bytes."""
    if x2d.dtype != torch.bfloat16 or not x2d.is_cuda or x2d.dim() != 2:
        return False
    M, C = x2d.shape
    shape_ok = C % 256 == 0 and H % 128 == 0 and 128 <= H <= 1024 and E <= 128 and E % 4 == 0 and k <= min(8, E)
    if M == 0:
        return shape_ok
    return (shape_ok and x2d.stride(-1) == 1 and x2d.stride(0) % 8 == 0 and x2d.data_ptr() % 16 == 0
            and M * x2d.stride(0) * 2 < 2 ** 31)


def moe_router_wide(x2d: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, E: int, k: int, dense: bool = False,
                    y: torch.Tensor = None, return_hidden: bool = False):
    """HadamardRouter.forward (moe.py:418-447) of a wide bf16 model on matrix
    cores: h = silu(x W1^T), logits = h W2^T, softmax / top-k / routing
    outputs.  x2d [M, C] bf16 (moe_router_wide_supported), w1 [H, C] and w2
    [E, H] bf16 contiguous.  If y [M, 32E] is given, the blocks of unselected
    experts are zeroed.  ``return_hidden`` also returns silu(x W1^T) [M, H]."""
    _hip.require_device(x2d, "input")
    assert w1.dtype == torch.bfloat16 and w2.dtype == torch.bfloat16 and w1.is_contiguous() and w2.is_contiguous()
    M, C = x2d.shape
    H = w1.shape[0]
    r = MoERoute(M, E, k, x2d.device, dense, _parts(M, 64 if M > 256 else 1, x2d.device))
    nws = _hip.lib().walsh_moe_router_wide_workspace_bytes(M, H, E)
    work = torch.empty(max(nws, 256), device=x2d.device, dtype=torch.uint8)
    ldy, ydt = 0, torch.bfloat16
    if y is not None:
        assert y.shape[-1] == 32 * E and y.stride(-1) == 1, "output layout"
        ldy, ydt = (y.stride(0) if y.dim() == 2 else 32 * E), y.dtype
    nbytes = M * C * 2 + (H * C + E * H) * 2 + 2 * M * H * 2 + M * k * 8
    if y is not None:
        nbytes += M * (E - k) * 32 * y.element_size()
    _hip.call("walsh_moe_router_wide_fwd", x2d.data_ptr(), x2d.stride(0) if M else C, M, C, H, w1.data_ptr(),
              w2.data_ptr(), E, k, work.data_ptr(), work.numel(), _hip.ptr(r.probs), _hip.ptr(r.mask),
              _hip.ptr(r.weights), r.topk_idx.data_ptr(), r.topk_w.data_ptr(), r.count_part.data_ptr(),
              r.probsum_part.data_ptr(), r.parts, _hip.ptr(y), ldy, _hip.dtype_code(ydt), _hip.stream(x2d.device),
              kernel="moe_router_wide<bf16>", nbytes=nbytes, flops=2 * M * (C * H + H * E))
    if return_hidden:
        return r, work[:M * H * 2].view(torch.bfloat16).view(M, H)
    return r


MOE_DECODE_MAX_TOKENS = 4


def moe_decode_supported(x2d: torch.Tensor, H: int, E: int, k: int, He: int, y: torch.Tensor) -> bool:
    """Whether walsh_moe_decode_fwd takes this MoE call: 1..4 tokens of a bf16
    wide model (the wide router's shapes with C == 32 E), expert hidden 64 /
    128 / 256, y with 16-byte-aligned rows."""
    M = x2d.shape[0] if x2d.dim() == 2 else 0
    return (1 <= M <= MOE_DECODE_MAX_TOKENS and x2d.shape[1] == 32 * E and He in (64, 128, 256)
            and moe_router_wide_supported(x2d, H, E, k) and y.is_cuda and y.dim() == 2 and y.stride(-1) == 1
            and y.dtype in (torch.bfloat16, torch.float32) and y.data_ptr() % 16 == 0
            and y.stride(0) % (16 // y.element_size()) == 0)


def moe_decode(x2d: torch.Tensor, y: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, E: int, k: int, frags,
               gammas: torch.Tensor, He: int, sync: torch.Tensor, dense: bool = False) -> MoERoute:
    """HadamardMoE.forward (moe.py:512-542) for a few tokens in one launch:
    routing (as moe_router_wide) and the routed experts (as moe_scatter +
    moe_experts) into y [M, 32E], bitwise their result.  sync: a one-element
    int32 device tensor that starts at zero (the kernel leaves it at zero);
    calls sharing it must not overlap."""
    _hip.require_device(x2d, "input")
    assert moe_decode_supported(x2d, w1.shape[0], E, k, He, y), "moe_decode shape"
    assert w1.dtype == torch.bfloat16 and w2.dtype == torch.bfloat16 and w1.is_contiguous() and w2.is_contiguous()
    assert sync.dtype == torch.int32 and sync.numel() >= 1 and sync.device == x2d.device
    M, C = x2d.shape
    H = w1.shape[0]
    r = MoERoute(M, E, k, x2d.device, dense, M)  # one partial row per token
    nws = _hip.lib().walsh_moe_decode_workspace_bytes(M, H, E)
    work = torch.empty(max(nws, 256), device=x2d.device, dtype=torch.uint8)
    gf, uf, df = frags
    g = gammas.detach().float().contiguous()
    nbytes = M * C * 2 + (H * C + E * H) * 2 + M * C * y.element_size() + M * k * 8 + 3 * E * He * 8
    _hip.call("walsh_moe_decode_fwd", x2d.data_ptr(), x2d.stride(0), M, C, H, w1.data_ptr(), w2.data_ptr(), E, k, He,
              gf.data_ptr(), uf.data_ptr(), df.data_ptr(), g.data_ptr(), work.data_ptr(), work.numel(),
              sync.data_ptr(), _hip.ptr(r.probs), _hip.ptr(r.mask), _hip.ptr(r.weights), r.topk_idx.data_ptr(),
              r.topk_w.data_ptr(), r.count_part.data_ptr(), r.probsum_part.data_ptr(), r.parts, y.data_ptr(),
              y.stride(0), _hip.dtype_code(y.dtype), _hip.stream(x2d.device), kernel="moe_decode<bf16>",
              nbytes=nbytes, flops=2 * M * (C * H + H * E) + 2 * M * k * 3 * 32 * He)
    return r


def moe_topk(logits: torch.Tensor, k: int, dense: bool = False) -> MoERoute:
    """Softmax / top-k / renormalisation (moe.py:432-445) on float32 logits [M, E]."""
    _hip.require_device(logits, "logits")
    lg = logits.detach().float().contiguous()
    M, E = lg.shape
    # partial-count rows: one per workgroup (16 tokens per wave up to 16
    # experts; one token per wave, 8 per workgroup, above)
    r = MoERoute(M, E, k, lg.device, dense, _parts(M, 64 if E <= 16 else 8, lg.device))
    _hip.call("walsh_moe_topk_fwd", lg.data_ptr(), M, E, k, _hip.ptr(r.probs), _hip.ptr(r.mask),
              _hip.ptr(r.weights), r.topk_idx.data_ptr(), r.topk_w.data_ptr(), r.count_part.data_ptr(),
              r.probsum_part.data_ptr(), r.parts, _hip.stream(lg.device), kernel="moe_topk_kernel",
              nbytes=M * E * 4 + M * k * 8)
    return r


def moe_scatter(r: MoERoute):
    """Per-expert pair lists: (list [M*k], offset [E+1], tile_off [E+1]) int32;
    also sets the totals r.count / r.probsum."""
    dev = r.topk_idx.device
    E = r.E
    lst = torch.empty(max(r.M * r.k, 1), device=dev, dtype=torch.int32)
    ints = torch.empty(4 * E + 2, device=dev, dtype=torch.int32)
    count, cursor, offset, tile_off = ints[:E], ints[E:2 * E], ints[2 * E:3 * E + 1], ints[3 * E + 1:]
    probsum = torch.empty(E, device=dev, dtype=torch.float32)
    _hip.call("walsh_moe_scatter", r.topk_idx.data_ptr(), r.M, E, r.k, r.count_part.data_ptr(),
              r.probsum_part.data_ptr(), r.parts, count.data_ptr(), probsum.data_ptr(), cursor.data_ptr(),
              lst.data_ptr(), offset.data_ptr(), tile_off.data_ptr(), _hip.stream(dev), kernel="moe_scatter_kernel",
              nbytes=r.M * r.k * 8)
    r._count, r._probsum = count, probsum
    return lst, offset, tile_off


def moe_experts(x: torch.Tensor, y: torch.Tensor, r: MoERoute, lists, frags, gammas: torch.Tensor, H: int):
    """Routed ternary SwiGLU experts (moe.py:337-380) for the pairs of ``r``:
    writes y[t, 32e:32e+32] for every selected (t, e).  x [M, 32E] and y
    [M, 32E] with unit inner stride; frags from moe_expert_fragments."""
    _hip.require_device(x, "input")
    E = r.E
    xv, M, ldx = _rows_view(x, 32 * E)
    assert M == r.M and y.shape[-1] == 32 * E and y.stride(-1) == 1, "expert input/output layout"
    ldy = y.stride(0) if y.dim() == 2 else 32 * E
    lst, offset, tile_off = lists
    gf, uf, df = frags
    g = gammas.detach().float().contiguous()
    esz, ysz = x.element_size(), y.element_size()
    pairs = M * r.k
    nbytes = pairs * 32 * (esz + ysz) + pairs * 8 + 3 * E * H * 8
    tag = "bf16" if x.dtype == torch.bfloat16 else "f32"
    _hip.call("walsh_moe_experts_fwd", xv.data_ptr(), ldx, y.data_ptr(), ldy, M, E, r.k, H, gf.data_ptr(),
              uf.data_ptr(), df.data_ptr(), g.data_ptr(), lst.data_ptr(), offset.data_ptr(), tile_off.data_ptr(),
              r.count.data_ptr(), r.topk_w.data_ptr(), _hip.dtype_code(x.dtype), _hip.dtype_code(y.dtype),
              _hip.stream(x.device), kernel="moe_experts_kernel<%s>" % tag, nbytes=nbytes,
              flops=2 * pairs * 3 * 32 * H)


def moe_experts_bwd(x: torch.Tensor, dout: torch.Tensor, r: MoERoute, lists, packed, gammas: torch.Tensor,
                    H: int, need_w: bool = True):
    """Backward of the routed experts (moe.py:337-380 with the MoE STE) over
    the pairs of ``r``: returns (dx [M, 32E] float32 with zeros outside the
    routed blocks, d_pair_w [M, k], (dgate, dup, ddown) or None).  x, dout
    [M, 32E] float32; packed = (gate, up, down) 2-bit codes; gammas [3]."""
    _hip.require_device(x, "input")
    E, k = r.E, r.k
    xv, M, ldx = _rows_view(x, 32 * E)
    dv, Md, ldd = _rows_view(dout, 32 * E)
    assert M == r.M == Md and x.dtype == torch.float32 and dout.dtype == torch.float32, "expert operands"
    lst, offset, _ = lists
    pg, pu, pd = (t.contiguous() for t in packed)
    dev = x.device
    dx = torch.zeros(M, 32 * E, device=dev, dtype=torch.float32)
    dpair = torch.empty(max(M * k, 1), device=dev, dtype=torch.float32)
    grads = tuple(torch.empty(sh, device=dev, dtype=torch.float32) for sh in ((E, H, 32), (E, H, 32), (E, 32, H))) \
        if need_w else (None, None, None)
    nws = _hip.lib().walsh_moe_experts_bwd_workspace_bytes(E, H)
    ws = torch.empty(max(nws, 4), device=dev, dtype=torch.uint8)
    g = gammas.detach().float().contiguous()
    _hip.call("walsh_moe_experts_bwd", xv.data_ptr(), ldx, dv.data_ptr(), ldd, M, E, k, H, pg.data_ptr(),
              pu.data_ptr(), pd.data_ptr(), g.data_ptr(), lst.data_ptr(), offset.data_ptr(), r.topk_w.data_ptr(),
              dx.data_ptr(), 32 * E, dpair.data_ptr(), *[_hip.ptr(t) for t in grads], ws.data_ptr(), ws.numel(),
              _hip.stream(dev), kernel="moe_experts_bwd_kernel", nbytes=M * k * 32 * 16 + 3 * E * H * 32 * 4,
              flops=2 * M * k * 32 * H * 9)
    return dx, dpair[:M * k].view(M, k), (grads if need_w else None)


def moe_ffn_supported(x2d: torch.Tensor, E: int, H: int, k: int) -> bool:
    """Whether walsh_moe_ffn_fwd (single-launch MoE) handles this call."""
    return (x2d.dtype == torch.bfloat16 and x2d.shape[-1] == 512 and E == 16 and H in (64, 128) and 1 <= k <= 8)


def moe_ffn_fragments(w1: torch.Tensor, w2: torch.Tensor, gate_packed: torch.Tensor, up_packed: torch.Tensor,
                      down_packed: torch.Tensor):
    """Operand layouts of walsh_moe_ffn_fwd from the router weights and the
    packed expert codes."""
    H1, C = w1.shape
    E, H = gate_packed.shape[0], gate_packed.shape[1]
    f1 = w1.detach().to(torch.bfloat16).reshape(H1 // 16, 16, C // 32, 4, 8).permute(0, 2, 3, 1, 4).contiguous()
    w2p = torch.zeros(16, H1, device=w2.device, dtype=torch.bfloat16)
    w2p[:E] = w2.detach().to(torch.bfloat16)
    f2 = w2p.reshape(16, H1 // 16, 4, 4).permute(1, 2, 0, 3).contiguous()  # [c][kq][m][s]

    def gu(p):  # [E][nt][m][kq][2] -> [E][kq][m][nt][2]
        return p.reshape(E, H // 16, 16, 4, 2).permute(0, 3, 2, 1, 4).contiguous().view(torch.int16)

    # [E][mt][m][c][half][kq] -> [E][kq][m][mt][c][half]
    dn = down_packed.reshape(E, 2, 16, H // 32, 2, 4).permute(0, 5, 2, 1, 3, 4).contiguous().view(torch.int16)
    return f1, f2, gu(gate_packed), gu(up_packed), dn


def moe_ffn(x: torch.Tensor, y: torch.Tensor, frags, gammas: torch.Tensor, E: int, k: int, H: int) -> MoERoute:
    """Single-launch HadamardMoE forward (walsh_moe_ffn_fwd): writes y [M, 512]
    (float32 or bf16) and returns the routing (topk_idx, topk_w, count, probsum)."""
    _hip.require_device(x, "input")
    xv, M, ldx = _rows_view(x, x.shape[-1])
    C = x.shape[-1]
    assert y.shape[-1] == C and y.stride(-1) == 1, "output layout"
    ldy = y.stride(0) if y.dim() == 2 else C
    parts = max(1, min((M + 63) // 64, _hip.cu_count(x.device)))
    r = MoERoute(M, E, k, x.device, dense=False, parts=parts)
    f1, f2, gf, uf, df = frags
    g = gammas.detach().float().contiguous()
    nbytes = M * C * (2 + y.element_size()) + M * k * 8 + (f1.numel() + f2.numel()) * 2 + 3 * E * H * 8
    flops = 2 * M * (C * (C // 4) + (C // 4) * E) + 2 * M * k * 3 * 32 * H
    _hip.call("walsh_moe_ffn_fwd", xv.data_ptr(), ldx, M, C, f1.data_ptr(), f2.data_ptr(), E, k, H, gf.data_ptr(),
              uf.data_ptr(), df.data_ptr(), g.data_ptr(), r.topk_idx.data_ptr(), r.topk_w.data_ptr(),
              r.count_part.data_ptr(), r.probsum_part.data_ptr(), parts, y.data_ptr(), ldy, _hip.dtype_code(x.dtype),
              _hip.dtype_code(y.dtype), _hip.stream(x.device),
              kernel="moe_ffn_kernel<%s>" % ("f32out" if y.dtype == torch.float32 else "bf16out"), nbytes=nbytes,
              flops=flops)
    return r
