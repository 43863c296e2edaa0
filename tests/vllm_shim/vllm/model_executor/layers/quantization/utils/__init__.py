import torch


def replace_parameter(mod, name, new):
    old = getattr(mod, name)
    if isinstance(new, torch.nn.Parameter):
        p = new
    else:
        p = torch.nn.Parameter(new, requires_grad=False)
    for k, v in vars(old).items():
        if not k.startswith("_"):
            setattr(p, k, v)
    delattr(mod, name)
    mod.register_parameter(name, p)
