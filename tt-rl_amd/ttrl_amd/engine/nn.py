"""`Module`, `ModuleList`, `ModuleDict` (ttrl/engine/nn/module.py:25-189,
ttrl/engine/nn/containers.py:15-84): parameters are discovered by walking
attributes in definition order, named by attribute path, de-duplicated by
identity; checkpoints load in place after validating every key and shape;
`copy_from` hard-copies a same-structured module in place."""

from __future__ import annotations

from typing import Iterator

import numpy as np

from ttrl_amd.engine.autograd import Tensor
from ttrl_amd.engine.tensor import arena_of, copy_tensor_in_place, restore_in_place

__all__ = ["Module", "ModuleList", "ModuleDict"]


def _named_from(prefix: str, value, seen: set):
    if isinstance(value, Tensor):
        if value.requires_grad and id(value) not in seen:
            seen.add(id(value))
            yield prefix, value
    elif isinstance(value, Module):
        for name, child in value._slot_sources():
            yield from _named_from(f"{prefix}.{name}", child, seen)
    elif callable(getattr(value, "named_parameters", None)):
        for sub, param in value.named_parameters():
            if id(param) not in seen:
                seen.add(id(param))
                yield f"{prefix}.{sub}", param
    elif isinstance(value, (list, tuple)):
        for index, item in enumerate(value):
            yield from _named_from(f"{prefix}.{index}", item, seen)
    elif isinstance(value, dict):
        for key, item in value.items():
            yield from _named_from(f"{prefix}.{key}", item, seen)


def _serialises_own_state(module) -> bool:
    return type(module).state_dict is not Module.state_dict


def _slots_from(prefix: str, value, seen: set):
    if isinstance(value, Tensor):
        if value.requires_grad and id(value) not in seen:
            seen.add(id(value))
            return [(prefix, value)]
        return []
    if isinstance(value, Module):
        if _serialises_own_state(value):
            # One module in two slots (a shared trunk) checkpoints once
            # (ttrl/engine/nn/discovery.py:128-139).
            if id(value) in seen:
                return []
            seen.add(id(value))
            return [(prefix, value)]
        out = []
        for name, child in value._slot_sources():
            out.extend(_slots_from(f"{prefix}.{name}", child, seen))
        return out
    return []


class Module:
    """Base class; subclasses register Tensors and submodules as attributes."""

    def _slot_sources(self):
        return vars(self).items()

    def _walk(self) -> Iterator[tuple[str, Tensor]]:
        seen: set[int] = set()
        for name, value in self._slot_sources():
            yield from _named_from(name, value, seen)

    def named_parameters(self) -> Iterator[tuple[str, Tensor]]:
        yield from self._walk()

    def parameters(self) -> Iterator[Tensor]:
        for _, p in self._walk():
            yield p

    def zero_grad(self) -> None:
        for p in self.parameters():
            p.zero_grad()

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    def forward(self, *args, **kwargs):
        raise NotImplementedError

    def _state_slots(self):
        seen: set[int] = set()
        slots = []
        for name, value in self._slot_sources():
            slots.extend(_slots_from(name, value, seen))
        return slots

    def state_dict(self) -> dict[str, np.ndarray]:
        out: dict[str, np.ndarray] = {}
        for name, target in self._state_slots():
            if isinstance(target, Tensor):
                out[name] = target.numpy()
                continue
            for key, array in target.state_dict().items():
                out[f"{name}.{key}"] = array
        return out

    def load_state_dict(self, state: dict, device=None) -> None:
        slots = self._state_slots()
        reference = self.state_dict()
        got, expected = set(state.keys()), set(reference)
        if got != expected:
            raise ValueError(
                "load_state_dict: checkpoint keys do not match module "
                f"parameters (missing={sorted(expected - got)}, extra={sorted(got - expected)})"
            )
        for name, want in reference.items():
            shape = tuple(int(d) for d in np.asarray(state[name]).shape)
            if shape != want.shape:
                raise ValueError(
                    f"load_state_dict: shape mismatch for {name!r}: "
                    f"checkpoint has {shape}, parameter expects {want.shape}"
                )
        for name, target in slots:
            if isinstance(target, Tensor):
                restore_in_place(target.data, state[name])
                continue
            prefix = f"{name}."
            target.load_state_dict({k[len(prefix):]: v for k, v in state.items() if k.startswith(prefix)})

    def copy_from(self, other: "Module") -> None:
        """Hard-copy another module's parameters, in place (target sync)."""
        dst_named = list(self.named_parameters())
        src_named = list(other.named_parameters())
        if len(dst_named) != len(src_named):
            raise ValueError(
                f"copy_from: parameter count mismatch ({len(dst_named)} vs {len(src_named)}); "
                "target and source modules do not match"
            )
        for (dst_name, dst), (src_name, src) in zip(dst_named, src_named):
            if dst_name != src_name:
                raise ValueError(
                    f"copy_from: parameter name mismatch ({dst_name!r} vs {src_name!r}); "
                    "the two modules have different structure"
                )
            if tuple(dst.shape) != tuple(src.shape):
                raise ValueError(
                    f"copy_from: shape mismatch for {dst_name!r}: target {tuple(dst.shape)}, "
                    f"source {tuple(src.shape)}"
                )
        da = arena_of(p for _, p in dst_named)
        sa = arena_of(p for _, p in src_named)
        if da is not None and sa is not None and da.offsets == sa.offsets:
            da.data.copy_from(sa.data)  # one copy over the whole arena
            return
        for (_, dst), (_, src) in zip(dst_named, src_named):
            copy_tensor_in_place(dst, src)


class ModuleList(Module):
    """An ordered list of modules named "0", "1", ..."""

    def __init__(self, modules=()):
        self._items = list(modules)

    def _slot_sources(self):
        return [(str(i), m) for i, m in enumerate(self._items)]

    def append(self, module) -> "ModuleList":
        self._items.append(module)
        return self

    def __iter__(self):
        return iter(self._items)

    def __len__(self):
        return len(self._items)

    def __getitem__(self, i):
        return self._items[i]


class ModuleDict(Module):
    """Modules by name, in insertion order."""

    def __init__(self, modules=None):
        self._items = dict(modules or {})

    def _slot_sources(self):
        return list(self._items.items())

    def __getitem__(self, key):
        return self._items[key]

    def __contains__(self, key):
        return key in self._items

    def keys(self):
        return self._items.keys()

    def items(self):
        return self._items.items()

    def values(self):
        return self._items.values()

    def __len__(self):
        return len(self._items)
