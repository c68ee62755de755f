"""Warmup-only launch choices, frozen before graph capture (engine/kernels/tune.py:1-48).

Same registry as the reference: ``pick`` returns the current option for a key
(registering it on first use, never selecting during capture), ``register``
records a ``Knob`` that a captured decode step may re-judge, ``knobs(rows)``
lists the knobs of one batch size, largest expected effect first.
"""

import torch

_BEST = {}
_KNOBS = {}


class Knob:
    """One frozen-at-warmup choice that the captured decode step can re-judge."""

    def __init__(self, name, rows, weight, options, get, select):
        self.name, self.rows, self.weight = name, rows, weight
        self.options, self.get, self.select = options, get, select


def register(name, rows, weight, options, get, select):
    _KNOBS[name] = Knob(name, rows, weight, options, get, select)


def knobs(rows):
    """Knobs of this batch size, largest expected effect first."""
    return sorted((knob for knob in _KNOBS.values() if knob.rows == rows), key=lambda knob: -knob.weight)


def pick(key, default, options, launch=None):
    """The current launch option for ``key``; registered on first use, outside capture."""
    if key not in _BEST:
        if torch.cuda.is_current_stream_capturing():
            return default
        _BEST[key] = default
        register(key, key[1], 1, [default, *[option for option in options if option != default]],
                 lambda: _BEST[key], lambda option: _BEST.__setitem__(key, option))
    return _BEST[key]
