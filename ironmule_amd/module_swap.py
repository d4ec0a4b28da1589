"""Swapping projections inside a torch module tree, and swapping them back.

The K=3840 admission (`qmv_k3840.enable`) and the geometry variant (`qmv_variant.install`)
both replace some `QuantizedLinear` children of a model with a module that serves
single-row decode from a gfx950 kernel and hands every other call to the module it
replaced.  They share three steps, kept here so that both follow them the same way:

1. `find_sites` lists every place in the tree where a candidate sits, as a `Site`
   (parent, attribute, dotted path, module), without changing anything;
2. the caller decides on every site (format checks, a probe) while the tree is untouched,
   so a refusal needs no undo;
3. `replace` installs the replacements; `restore` later puts the originals back by
   attribute, so the model holds the very objects it held before.

A replacement is a `DecodeOverride`.  It keeps the original module as a plain attribute,
outside the module tree, so a later walk (or `named_modules`) sees one projection per
site, and it shares the original's weight, scale and bias tensors rather than copying.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Iterator, Sequence

import torch


@dataclass(frozen=True, eq=False)
class Site:
    """One child slot of the tree: `getattr(parent, name)` is `module`."""

    parent: torch.nn.Module
    name: str
    path: str
    module: torch.nn.Module


def find_sites(root: torch.nn.Module, match: Callable[[torch.nn.Module], bool], *,
               opaque: tuple[type, ...] = ()) -> list[Site]:
    """Every child under `root` for which `match` holds, in declaration order.

    A matching child is not searched further; neither is an instance of an `opaque` type
    (a replacement already installed, whose original must stay hidden)."""

    def visit(parent: torch.nn.Module, prefix: str) -> Iterator[Site]:
        for name, child in parent.named_children():
            path = prefix + name
            if opaque and isinstance(child, opaque):
                continue
            if match(child):
                yield Site(parent, name, path, child)
            else:
                yield from visit(child, path + ".")

    return list(visit(root, ""))


def replace(sites: Sequence[Site], make: Callable[[torch.nn.Module], torch.nn.Module]) -> None:
    """Put `make(site.module)` into every site."""
    for site in sites:
        setattr(site.parent, site.name, make(site.module))


def restore(root: torch.nn.Module, kind: type) -> list[str]:
    """Put back the original of every `kind` replacement under `root`; their paths."""
    sites = find_sites(root, lambda m: isinstance(m, kind))
    for site in sites:
        setattr(site.parent, site.name, site.module.original)
    return [site.path for site in sites]


def in_features(module: torch.nn.Module) -> int:
    """The reduction length of a packed projection: 32-bit words times values per word."""
    return int(module.weight.shape[-1]) * 32 // int(module.bits)


class DecodeOverride(torch.nn.Module):
    """A projection whose single-token decode call, x of shape (1, 1, K), runs `decode`
    and whose every other call runs the module it replaced, on the same tensors.

    Subclasses implement `decode(row)` for a (1, K) row and may narrow `serves(x)`."""

    def __init__(self, original: torch.nn.Module) -> None:
        super().__init__()
        # A plain instance attribute, not a registered submodule (see the module text).
        self.__dict__["original"] = original
        self.weight = original.weight
        self.scales = original.scales
        self.biases = original.biases
        self.group_size = original.group_size
        self.bits = original.bits
        self.out_features = int(original.weight.shape[0])

    def serves(self, x: torch.Tensor) -> bool:
        return x.dim() == 3 and x.shape[0] == 1 and x.shape[1] == 1

    def decode(self, row: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self.serves(x):
            return self.original(x)
        y = self.decode(x[0]).unsqueeze(0)
        bias = getattr(self.original, "bias", None)
        return y if bias is None else y + bias
