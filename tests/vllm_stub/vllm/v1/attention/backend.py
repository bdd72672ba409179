import enum


class AttentionType(str, enum.Enum):
    DECODER = "decoder"
    ENCODER = "encoder"
    ENCODER_ONLY = "encoder_only"
    ENCODER_DECODER = "encoder_decoder"


class MultipleOf:
    def __init__(self, base):
        self.base = base


class AttentionBackend:
    pass


class AttentionImpl:
    pass


class AttentionLayer:
    pass


class AttentionMetadata:
    pass


class AttentionMetadataBuilder:
    pass
