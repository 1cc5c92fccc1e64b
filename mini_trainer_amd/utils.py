"""Installation helper with the reference's plugin mechanism."""
from __future__ import annotations

import importlib
from typing import Any


def patch_target_module(to_patch: str, replace_with: Any) -> None:
    """Replace the attribute named by a dotted path, e.g.
    "transformers.loss.loss_utils.fixed_cross_entropy".

    Same contract as the reference's utils.py:36-46: everything before the
    last dot is imported as a module and the last component is set on it.
    Callers that look the name up in module globals at call time (as
    TF/loss/loss_utils.py:70 does) then reach the replacement.
    """
    parts = to_patch.split(".")
    assert len(parts) > 1, "must have an object to patch"
    module = importlib.import_module(".".join(parts[:-1]))
    setattr(module, parts[-1], replace_with)
