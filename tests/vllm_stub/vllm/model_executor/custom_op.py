op_registry = {}
op_registry_oot = {}
