import torch


class LinearMethodBase:
    def create_weights(self, *args, **kwargs):
        raise NotImplementedError

    def apply(self, layer, x, bias=None):
        raise NotImplementedError

    def process_weights_after_loading(self, layer):
        return None


class LinearBase(torch.nn.Module):
    def __init__(self, tp_size=1):
        super().__init__()
        self.tp_size = tp_size
