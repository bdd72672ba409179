def set_weight_attrs(weight, weight_attrs):
    for key, value in (weight_attrs or {}).items():
        setattr(weight, key, value)
