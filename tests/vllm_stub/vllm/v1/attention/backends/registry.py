import enum

REGISTERED = {}


class AttentionBackendEnum(enum.Enum):
    CUSTOM = "CUSTOM"


def register_backend(backend, class_path=None):
    REGISTERED[backend] = class_path
