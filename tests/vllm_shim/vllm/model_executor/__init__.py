import torch


class PackedvLLMParameter(torch.nn.Parameter):
    """Parameter carrying vLLM's packing metadata and weight loader."""

    def __new__(cls, data, input_dim, output_dim, packed_dim, packed_factor, weight_loader):
        p = super().__new__(cls, data, requires_grad=False)
        p.input_dim = input_dim
        p.output_dim = output_dim
        p.packed_dim = packed_dim
        p.packed_factor = packed_factor
        p.weight_loader = weight_loader
        return p
