def set_weight_attrs(weight, weight_attrs):
    for k, v in (weight_attrs or {}).items():
        setattr(weight, k, v)
