class QuantizeMethodBase:
    pass


class QuantizationConfig:
    def __init__(self):
        self.packed_modules_mapping = {}
