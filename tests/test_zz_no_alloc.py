"""The allocation-free variant of the source preparation (mkx_source_run_noalloc), through the C ABI: two
calls in a row, the second with a smaller context, each equal bit for bit to mkx_source_run on the same
inputs (the static array keeps the first call's staging, which the second must not read), and a context
too large for the static array refused before any launch."""
import pytest
import torch

from mkx import _lib, synthetic as SY
from mkx._lib import MkxError
from mkx.prepare import SourcePrepare

pytestmark = pytest.mark.gpu
torch.set_grad_enabled(False)


def _same(a, b):
    return all(torch.equal(ka, kb) and torch.equal(va, vb) for (ka, va), (kb, vb) in zip(a, b))


def test_static_scratch_source_preparation_matches_the_allocating_one():
    cfg = SY.WORKLOADS["A"]
    model = SY.SyntheticReki(cfg, SY.make_weights(cfg, 0), device="cuda")
    prep = SourcePrepare(model)
    g = torch.Generator().manual_seed(5)
    big = torch.randn(2, 300, cfg.ctx_dim, generator=g).to(torch.bfloat16).cuda()
    small = torch.randn(1, 70, cfg.ctx_dim, generator=g).to(torch.bfloat16).cuda()
    big_len = torch.tensor([300, 211], dtype=torch.int32, device="cuda")
    small_len = torch.tensor([70], dtype=torch.int32, device="cuda")
    na_big = prep(big, big_len, static_scratch=True)
    na_small = prep(small, small_len, static_scratch=True)  # smaller: must not read the first call's staging
    torch.cuda.synchronize()
    ref_big = prep(big, big_len)
    ref_small = prep(small, small_len)
    torch.cuda.synchronize()
    assert _same(na_big, ref_big), "first call differs from mkx_source_run"
    assert _same(na_small, ref_small), "second, smaller call differs from mkx_source_run"
    assert all(bool(torch.isfinite(k.float()).all()) for k, _ in na_small)
    # a packed context above the static array's 16 MiB is refused (4160 rows x 2048 x 2 bytes)
    too_big = torch.zeros(1, 4100, cfg.ctx_dim, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(MkxError) as ei:
        prep(too_big, torch.tensor([4100], dtype=torch.int32, device="cuda"), static_scratch=True)
    assert ei.value.status == _lib.EINVAL
    prep.close()
