class QuantizeMethodBase:
    def create_weights(self, layer, *args, **kwargs):
        raise NotImplementedError

    def apply(self, layer, *args, **kwargs):
        raise NotImplementedError

    def process_weights_after_loading(self, layer):
        return None


class QuantizationConfig:
    def __init__(self):
        self.packed_modules_mapping = {}
