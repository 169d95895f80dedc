"""Stand-in for comfy_api.latest (ComfyExtension and the io schema types), for tests only."""


class ComfyExtension:
    pass


class _Input:
    def __init__(self, name, **kwargs):
        self.name = name
        self.kwargs = kwargs


class _Type:
    Input = _Input

    @staticmethod
    def Output(*args, **kwargs):
        return ("output", args, kwargs)


class io:
    class ComfyNode:
        pass

    class Schema:
        def __init__(self, **kwargs):
            self.__dict__.update(kwargs)

    class NodeOutput(tuple):
        def __new__(cls, *values):
            return super().__new__(cls, values)

    Model = _Type
    Float = _Type
    Int = _Type
    Boolean = _Type
    Combo = _Type
    String = _Type
