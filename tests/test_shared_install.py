"""moe/shared.install binds the fused forward only on gated shared-expert MLPs, and the bound forward falls back to
the stock one when the projections are not on the MXFP4 kernels (no GPU needed: the fallback path runs on the CPU)."""
import torch

from r9700_vllm.moe import shared


class UnquantizedLinearMethod:                # stands in for vLLM's class of that name
    pass


class _Gate(torch.nn.Module):
    def __init__(self, H, bias=False):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.zeros(1, H, dtype=torch.bfloat16), requires_grad=False)
        self.bias = torch.nn.Parameter(torch.zeros(1)) if bias else None
        self.quant_method = UnquantizedLinearMethod()


class Qwen3NextMLP(torch.nn.Module):          # the module class name the hook matches
    def __init__(self, H, gate=True, bias=False):
        super().__init__()
        self.gate_up_proj = torch.nn.Linear(H, 2 * H, bias=False)
        self.down_proj = torch.nn.Linear(H, H, bias=False)
        if gate:
            self.expert_gate = _Gate(H, bias)

    def forward(self, x):
        return x + 1


def test_install_binds_gated_mlps_and_falls_back():
    model = torch.nn.ModuleDict({"a": Qwen3NextMLP(8), "b": Qwen3NextMLP(8, gate=False),
                                 "c": Qwen3NextMLP(8, bias=True), "d": torch.nn.Linear(8, 8)})
    n = shared.install(model)
    assert n == 1 and getattr(model["a"], "_r9k_shared", False) and not getattr(model["c"], "_r9k_shared", False)
    assert shared.install(model) == 0                                  # idempotent
    x = torch.zeros(2, 8, dtype=torch.bfloat16)
    assert torch.equal(model["a"](x), x + 1)                           # projections not prepared: stock forward
