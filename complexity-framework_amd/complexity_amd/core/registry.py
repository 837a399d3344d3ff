"""Name -> class registry for MLP plug-ins (behaviour of complexity/core/registry.py).

``MLP_REGISTRY.build(name, config)`` is how a transformer block instantiates
its feed-forward (block.py:203); ``register_mlp`` is the decorator plug-ins use.
"""

from __future__ import annotations

from typing import Callable, Dict, Type


class Registry:
    def __init__(self, kind: str):
        self.kind = kind
        self._entries: Dict[str, Type] = {}

    def register(self, name: str) -> Callable[[Type], Type]:
        def decorate(cls: Type) -> Type:
            self._entries[name] = cls
            return cls

        return decorate

    def get(self, name: str) -> Type:
        try:
            return self._entries[name]
        except KeyError:
            raise KeyError(f"unknown {self.kind} {name!r}; registered: {sorted(self._entries)}") from None

    def build(self, name: str, *args, **kwargs):
        return self.get(name)(*args, **kwargs)

    def list(self):
        return sorted(self._entries)

    def __contains__(self, name: str) -> bool:
        return name in self._entries


MLP_REGISTRY = Registry("mlp")


def register_mlp(name: str):
    return MLP_REGISTRY.register(name)
