import torch


class ModelWeightParameter(torch.nn.Parameter):
    def __new__(cls, data, input_dim=None, output_dim=None, weight_loader=None):
        p = super().__new__(cls, data, requires_grad=False)
        p.input_dim, p.output_dim, p.weight_loader = input_dim, output_dim, weight_loader
        return p
