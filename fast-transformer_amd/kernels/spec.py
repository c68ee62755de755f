"""Speculative verify-block bookkeeping (engine/kernels/spec.py): outside this library.

The reference drafts several tokens per row and verifies them in one pass
(engine/decode.py:425-475, engine/kernels/spec.py). That path, with the
verify-block attention it needs (engine/kernels/decode_attention.py:637-680
``block_attention``), is not part of the decode path this library implements.
The names exist so that engine code importing them loads; calling one raises.
One-token decode steps need none of them: the reference's DecodeState takes
that path when the model has no ``successor`` table (engine/decode.py:295), and
this package's ``decode.Decoder`` always does.
"""

_WHY = ("speculative verify blocks (engine/kernels/spec.py) are outside this library; decode one token "
        "per step (a model without `successor`, or decode.Decoder)")


def propose(history, position, tokens_per_row, drafts_by_match, successor, stale, chains, phases):
    """engine/kernels/spec.py:106-125. Raises NotImplementedError."""
    raise NotImplementedError(_WHY)


def within_margin(logits, tokens, top, margin):
    """engine/kernels/spec.py:154-167. Raises NotImplementedError."""
    raise NotImplementedError(_WHY)


def settle(tokens, greedy, position, limit, history, result, move_from, move_to, chains, stale, within=None):
    """engine/kernels/spec.py:227-241. Raises NotImplementedError."""
    raise NotImplementedError(_WHY)


def relocate(store, move_from, move_to):
    """engine/kernels/spec.py:262-270. Raises NotImplementedError."""
    raise NotImplementedError(_WHY)
