QUANTIZATION_METHODS = {}


def register_quantization_config(name):
    def deco(cls):
        QUANTIZATION_METHODS[name] = cls
        return cls
    return deco
