"""Weights derived from module parameters (the concatenated Q/K/V projection,
the interleaved gate/up projection), kept in step with their sources.

The reference's modules read their nn.Linear weights on every call
(torchpp/attention/gqa.py:82-84, examples/LLM/fastqwen3.py:71-78), so a
`load_state_dict` or an in-place edit of a weight takes effect on the next
forward. A derived copy has to follow the same contract: it is keyed on each
source's storage address, version counter, dtype and shape, and rebuilt when
any of them changes. A module that owns one also invalidates it from a
load_state_dict post-hook, which covers inference tensors (they carry no
version counter).

A rebuild writes into the existing buffer when shape, dtype and device are
unchanged, so a HIP graph captured on the old buffer reads the new weights
on its next replay. A rebuild requested while the current stream is being
captured is recorded into the graph and not cached: its values exist only
once the graph has run.
"""
from __future__ import annotations

from typing import Callable, Optional

import torch


def _version(t: torch.Tensor) -> Optional[int]:
    try:
        return t._version
    except RuntimeError:  # inference tensors have no version counter
        return None


def _key(t: torch.Tensor):
    return (t.data_ptr(), _version(t), t.dtype, tuple(t.shape), t.device)


class DerivedWeight:
    def __init__(self, build: Callable[..., torch.Tensor]):
        self._build = build
        self._key = None
        self._buf: Optional[torch.Tensor] = None

    def invalidate(self) -> None:
        self._key = None

    def get(self, *sources: torch.Tensor) -> torch.Tensor:
        key = tuple(_key(t) for t in sources)
        if key == self._key and self._buf is not None:
            return self._buf
        capturing = sources[0].is_cuda and torch.cuda.is_current_stream_capturing()
        with torch.inference_mode(False), torch.no_grad():
            new = self._build(*sources)
            if capturing:
                return new
            buf = self._buf
            if (buf is not None and buf.shape == new.shape and buf.dtype == new.dtype
                    and buf.device == new.device):
                buf.copy_(new)
            else:
                self._buf = new
        self._key = key
        return self._buf


def _invalidate_all(module: torch.nn.Module, incompatible_keys) -> None:
    for v in vars(module).values():
        if isinstance(v, DerivedWeight):
            v.invalidate()


def attach(module: torch.nn.Module, derived: DerivedWeight) -> DerivedWeight:
    """Have a state-dict load into `module` invalidate every DerivedWeight
    attribute of `module` (the hook looks them up on the module it is called
    for, so copies of the module invalidate their own)."""
    if not getattr(module, "_derived_hook", False):
        module.register_load_state_dict_post_hook(_invalidate_all)
        module._derived_hook = True
    return derived
