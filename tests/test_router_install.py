"""router.install binds the op only on `mlp.gate` modules that are unquantized bf16 linears without bias, and the
bound forward is the op's (no GPU needed: the op's fake gives its shapes on meta tensors, and router_gemm sends CPU
tensors to torch's GEMM)."""
import torch
import torch.nn.functional as F

from r9700_vllm import router as R


class UnquantizedLinearMethod:                # stand-ins for vLLM's classes of these names
    pass


class Fp8LinearMethod:
    pass


class ReplicatedLinear(torch.nn.Module):
    def __init__(self, E, H, bias=False, quant=UnquantizedLinearMethod, dtype=torch.bfloat16):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.randn(E, H).to(dtype), requires_grad=False)
        self.bias = torch.nn.Parameter(torch.zeros(E)) if bias else None
        self.quant_method = quant()
        self.return_bias = True

    def forward(self, x):
        return "stock", None


class Block(torch.nn.Module):
    def __init__(self, gate):
        super().__init__()
        self.mlp = torch.nn.Module()
        self.mlp.gate = gate


def test_install_binds_plain_bf16_gates_only():
    layers = torch.nn.ModuleList([Block(ReplicatedLinear(16, 32)), Block(ReplicatedLinear(16, 32, bias=True)),
                                  Block(ReplicatedLinear(16, 32, quant=Fp8LinearMethod)),
                                  Block(ReplicatedLinear(16, 32, dtype=torch.float32)), Block(torch.nn.Linear(32, 16))])
    assert R.install(layers) == 1
    assert getattr(layers[0].mlp.gate, "_r9k_router", False)
    assert all(not getattr(b.mlp.gate, "_r9k_router", False) for b in layers[1:])
    assert R.install(layers) == 0                                          # idempotent
    assert layers[0].mlp.gate.forward.__func__ is R._forward
    assert layers[1].mlp.gate(None)[0] == "stock"
    xm = torch.empty(3, 32, dtype=torch.bfloat16, device="meta")
    wm = torch.empty(16, 32, dtype=torch.bfloat16, device="meta")
    o = torch.ops.r9700.router_gemm(xm, wm, True)
    assert o.shape == (3, 16) and o.dtype == torch.bfloat16
    assert torch.ops.r9700.router_gemm(xm, wm, False).dtype == torch.float32
    x = torch.randn(3, 32).to(torch.bfloat16)
    w = layers[0].mlp.gate.weight
    assert torch.equal(R.router_gemm(x, w, True), F.linear(x, w))


def test_install_off_by_env(monkeypatch):
    monkeypatch.setenv("R9K_ROUTER", "stock")
    assert R.install(torch.nn.ModuleList([Block(ReplicatedLinear(16, 32))])) == 0
