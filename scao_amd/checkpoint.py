"""Loading SCAO checkpoints with torch's safe loader.

The optimizer's ``state_dict()`` keeps each parameter's live preconditioner
object in its per-parameter state (the reference inherits this from
``torch.optim.Optimizer``, scao/optimizer.py:732-756), so a checkpoint file
pickles that class: ``scao.preconditioner.SparsePreconditioner`` when the
reference wrote it, ``scao_amd.preconditioner.SparsePreconditioner`` when this
package did.  Every other object in such a file is one that
``torch.load(weights_only=True)`` already accepts.

``load`` runs ``torch.load(weights_only=True)`` with both names allow-listed:
this package's class, and for the reference's name a data-only record that
keeps the pickled attributes and executes nothing.  ``SCAO.load_state_dict``
then rebuilds a preconditioner for each parameter, takes its numbers from the
portable ``_scao_precond`` entry, and the diagonal bias factor (which only
the object carries) from the record.
"""

from __future__ import annotations

import torch

from .preconditioner import SparsePreconditioner


class ReferencePreconditionerRecord:
    """The attributes of a pickled ``scao.preconditioner.SparsePreconditioner``
    (scao/preconditioner.py:72-239), as data."""

    def __setstate__(self, state: dict) -> None:
        self.__dict__.update(state)


# the name the reference's pickles carry, so the safe loader maps it here
ReferencePreconditionerRecord.__module__ = "scao.preconditioner"
ReferencePreconditionerRecord.__name__ = "SparsePreconditioner"
ReferencePreconditionerRecord.__qualname__ = "SparsePreconditioner"

SAFE_GLOBALS = [ReferencePreconditionerRecord, SparsePreconditioner]


def load(f, map_location=None):
    """``torch.load(f, map_location, weights_only=True)`` for a checkpoint
    written by ``SCAO.state_dict()`` of the reference or of this package."""
    with torch.serialization.safe_globals(SAFE_GLOBALS):
        return torch.load(f, map_location=map_location, weights_only=True)
