"""WeightCache change detection (host logic, CPU only).

The layers cache derived weight layouts (ternary codes, kernel fragments)
keyed on each parameter's storage pointer, autograd version counter, shape,
dtype and device, plus a global epoch.  In-place writes on the parameter and
optimizer steps bump the version counter; a write through ``.data`` does
not, so ``invalidate_weight_caches()`` (or ``mHCWalsh.invalidate_weight_caches``)
must follow one.
"""
import torch

from src.model._common import WeightCache, invalidate_weight_caches


def test_weight_cache_detects_versions_and_needs_invalidate_after_data_writes():
    p = torch.nn.Parameter(torch.randn(8))
    cache = WeightCache()
    builds = []

    def build():
        builds.append(p.detach().clone())
        return builds[-1]

    a = cache.get([p], build)
    assert cache.get([p], build) is a and len(builds) == 1
    with torch.no_grad():
        p.mul_(2)                       # in-place on the parameter: version bump
    b = cache.get([p], build)
    assert len(builds) == 2 and torch.equal(b, p.detach())
    opt = torch.optim.SGD([p], lr=0.1)
    p.grad = torch.ones_like(p)
    opt.step()                          # optimizer step: version bump
    assert torch.equal(cache.get([p], build), p.detach()) and len(builds) == 3
    p.data.mul_(3)                      # .data write: invisible to the version counter
    stale = cache.get([p], build)
    assert len(builds) == 3 and not torch.equal(stale, p.detach())
    invalidate_weight_caches()
    assert torch.equal(cache.get([p], build), p.detach()) and len(builds) == 4


def test_load_state_dict_invalidates():
    lin = torch.nn.Linear(4, 4)
    cache = WeightCache()
    first = cache.get([lin.weight], lambda: lin.weight.detach().clone())
    lin.load_state_dict({"weight": torch.zeros(4, 4), "bias": torch.zeros(4)})
    again = cache.get([lin.weight], lambda: lin.weight.detach().clone())
    assert not torch.equal(first, again) and torch.equal(again, torch.zeros(4, 4))
