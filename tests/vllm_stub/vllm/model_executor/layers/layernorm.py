import torch


class RMSNorm(torch.nn.Module):
    """Dispatches like vLLM's CustomOp on ROCm: forward -> forward_hip."""

    def __init__(self, hidden_size, eps=1e-6, dtype=None, **_):
        super().__init__()
        self.hidden_size = hidden_size
        self.variance_epsilon = eps
        self.weight = torch.nn.Parameter(torch.ones(hidden_size, dtype=dtype), requires_grad=False)

    def forward_native(self, x, residual=None):
        raise AssertionError("stock RMSNorm reached")

    forward_cuda = forward_native
    forward_hip = forward_native

    def forward(self, x, residual=None):
        return self.forward_hip(x, residual)
