"""The committed TunableOp selections load on this software stack and the
products they select agree with the default heuristics' results."""
import pytest
import torch

from tagseq2tagseq_amd import gemm_tuning

pytestmark = pytest.mark.gpu


def test_tuned_selections_load_and_agree():
    g = torch.Generator().manual_seed(0)
    a = torch.randn(16384, 768, generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn(2304, 768, generator=g) * 0.03).to(torch.bfloat16).cuda()
    torch.cuda.tunable.enable(False)
    ref = a @ w.t()
    try:
        assert gemm_tuning.use_tuned_gemms()
        assert torch.cuda.tunable.is_enabled() and not torch.cuda.tunable.tuning_is_enabled()
        got = a @ w.t()
    finally:
        torch.cuda.tunable.enable(False)
    torch.testing.assert_close(got.float(), ref.float(), rtol=2e-2, atol=2e-2)
