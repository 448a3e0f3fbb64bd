"""TEST-ONLY: PluggableLayer with an out-of-tree registry."""


class PluggableLayer:
    oot_registry = {}

    @classmethod
    def register_oot(cls, _decorated_layer_cls=None, name=None):
        def deco(layer_cls):
            PluggableLayer.oot_registry[name or layer_cls.__name__] = layer_cls
            return layer_cls
        if _decorated_layer_cls is not None:
            return deco(_decorated_layer_cls)
        return deco
