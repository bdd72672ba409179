import torch


def _copy_loader(param, loaded):
    param.data.copy_(loaded)


class LinearBase(torch.nn.Module):
    """y = x W^T + b through the quant method, W [out, in] (vLLM layout)."""

    def __init__(self, input_size, output_size, bias=True, params_dtype=torch.bfloat16,
                 quant_config=None, prefix=""):
        super().__init__()
        self.quant_method = quant_config.get_quant_method(self, prefix)
        self.quant_method.create_weights(self, input_size, [output_size], input_size, output_size,
                                         params_dtype, weight_loader=_copy_loader)
        self.bias = torch.nn.Parameter(torch.zeros(output_size, dtype=params_dtype),
                                       requires_grad=False) if bias else None

    def forward(self, x):
        return self.quant_method.apply(self, x, self.bias)
