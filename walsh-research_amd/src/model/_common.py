"""Shared host-side helpers for the nn.Module layer."""
import torch


def act_dtype(x: torch.Tensor) -> torch.dtype:
    """Activation dtype the hot-path kernels compute in for input ``x``.

    Under ``torch.autocast('cuda', dtype=bf16)`` -- how the reference runs bf16
    (train.py:107, generate.py:134) -- it is the autocast dtype; otherwise the
    input's own dtype (float32 or bfloat16)."""
    if x.is_cuda and torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return x.dtype


def tracked_dtype(dt: torch.dtype) -> torch.dtype:
    """Compute dtype for batched products that autograd tracks: float32 in
    place of bfloat16.  The backward of a bf16 batched product multiplies by
    a transposed view of its right operand, a form of torch.bmm that has
    faulted the GPU here, so training-path batched products run in float32
    (their results are cast back to the activation dtype)."""
    return torch.float32 if dt == torch.bfloat16 else dt


_EPOCH = [0]


def invalidate_weight_caches() -> None:
    """Drop every cached weight derivative (ternary codes, packed kernel
    layouts, concatenated projections) of every module.

    Needed after a parameter is written in a way autograd's version counter
    does not see: through ``.data`` (``p.data.copy_(...)``,
    ``p.data.clamp_(...)``) or by another process or library writing its
    memory.  Optimizer steps, in-place writes on the parameter itself,
    ``load_state_dict`` and ``.to()`` are detected without it."""
    _EPOCH[0] += 1


class WeightCache:
    """Caches a device-side derivative of a parameter (its ternary codes,
    packed layouts, concatenations ...) until the parameter changes.

    The key is (data_ptr, _version, device, shape, dtype) plus a global
    epoch: an optimizer step bumps ``_version``, a ``.to()`` moves
    ``data_ptr``, and ``invalidate_weight_caches()`` bumps the epoch, so any
    of them rebuilds.  A write through ``.data`` bumps none of these: call
    ``invalidate_weight_caches()`` after one."""

    def __init__(self):
        self._key = None
        self._val = None

    def get(self, tensors, build, extra=()):
        key = tuple((t.data_ptr(), t._version, t.device, tuple(t.shape), t.dtype) for t in tensors) + tuple(extra)
        key = (_EPOCH[0],) + key
        if key != self._key:
            self._val = build()
            self._key = key
        return self._val

    def clear(self):
        self._key = None
        self._val = None


def cached_linear(mod: torch.nn.Linear, x: torch.Tensor, cache: WeightCache) -> torch.Tensor:
    """``mod(x)``, keeping autocast's cast of the weight and bias across calls.

    Under autocast F.linear casts the float32 weight and bias to the
    autocast dtype on every call (for the 50257 x 4096 output head that is a
    1.2 GB pass per call).  In inference (autograd off or nothing to track)
    the cast copies are kept in ``cache`` until a parameter changes; the
    product then sees exactly the operands autocast would have made."""
    dev = x.device.type
    if not (x.is_cuda and torch.is_autocast_enabled(dev)) or (
            torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in mod.parameters()))):
        return mod(x)
    dt = torch.get_autocast_dtype(dev)
    ps = (mod.weight,) if mod.bias is None else (mod.weight, mod.bias)
    cast = cache.get(ps, lambda: tuple(p.detach().to(dt) for p in ps), extra=(dt,))
    return torch.nn.functional.linear(x, cast[0], cast[1] if len(cast) > 1 else None)


def adjacent_parts_view(parts, width: int):
    """If ``parts`` are equal-shape slices laid side by side along the last
    dim of one tensor (what ``x.split(width, -1)`` returns), return the
    covering view without copying; otherwise None.  Also None when autograd
    tracks the parts: a view built from the first part's storage would not
    carry the other parts' gradients, so the caller concatenates."""
    if torch.is_grad_enabled() and any(p.requires_grad for p in parts):
        return None
    p0 = parts[0]
    if p0.shape[-1] != width or p0.stride(-1) != 1:
        return None
    esz = p0.element_size()
    base = p0.data_ptr()
    for i, p in enumerate(parts):
        if p.shape != p0.shape or p.stride() != p0.stride() or p.dtype != p0.dtype:
            return None
        if p.data_ptr() != base + i * width * esz:
            return None
    full = width * len(parts)
    if p0.dim() >= 2 and p0.stride(-2) < full:
        return None
    return torch.as_strided(p0, p0.shape[:-1] + (full,), p0.stride(), p0.storage_offset())
