"""Launch choices made during eager warmup and frozen before any graph is captured.

A *knob* is one such choice: a list of interchangeable launch options that all
compute the same values, a getter for the option in force and a setter. Nothing
here times anything. The timing lives with the callers: ``kernels.linear``
times candidate kinds once per shape at warmup, and ``kernels.linear.refine``
re-times each knob's alternatives inside a captured step and keeps an
alternative only when the whole step gets faster.

The public surface is that of engine/kernels/tune.py:13-48: ``Knob``,
``register``, ``knobs`` and ``pick``, with the same arguments and meaning.
"""

import torch

#: name -> Knob, in registration order (registering a name again replaces its knob).
_REGISTRY = {}
#: pick() key -> the option in force for it.
_IN_FORCE = {}


class Knob:
    """A warmup choice that a captured step may re-judge.

    ``options`` lists the interchangeable launch options, the warmup choice
    first; ``get()`` returns the option in force and ``select(option)`` puts
    another in force. ``rows`` is the batch size the choice belongs to, and
    ``weight`` orders re-judging: heavier knobs (more of the step's traffic)
    go first.
    """

    __slots__ = ("name", "rows", "weight", "options", "get", "select")

    def __init__(self, name, rows, weight, options, get, select):
        self.name = name
        self.rows = rows
        self.weight = weight
        self.options = list(options)
        self.get = get
        self.select = select

    def __repr__(self):
        return f"Knob({self.name!r}, rows={self.rows}, weight={self.weight}, {len(self.options)} options)"


def register(name, rows, weight, options, get, select):
    """Record the knob ``name`` (replacing an earlier knob of that name)."""
    _REGISTRY[name] = Knob(name, rows, weight, options, get, select)


def knobs(rows):
    """The knobs of batch size ``rows``, heaviest first (equal weights keep registration order)."""
    mine = [knob for knob in _REGISTRY.values() if knob.rows == rows]
    mine.sort(key=lambda knob: knob.weight, reverse=True)
    return mine


def pick(key, default, options, launch=None):
    """The launch option in force for ``key`` (``key[1]`` is its row count).

    The first call outside graph capture freezes ``default`` and registers a
    knob over ``default`` followed by the other ``options``, so a captured step
    can re-judge it later. A call during capture before that returns
    ``default`` and registers nothing. ``launch`` is accepted for the
    reference's signature; no option is timed here.
    """
    if key in _IN_FORCE:
        return _IN_FORCE[key]
    if torch.cuda.is_current_stream_capturing():
        return default
    _IN_FORCE[key] = default
    alternatives = [default] + [option for option in options if option != default]

    def current():
        return _IN_FORCE[key]

    def choose(option):
        _IN_FORCE[key] = option

    register(key, key[1], 1, alternatives, current, choose)
    return default
