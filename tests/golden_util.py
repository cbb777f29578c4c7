"""Golden-fixture helpers for the tests (restating the reference's fixture loaders).

``seeded_parameters`` restates ``tests/fixture_parameters.py:15-25`` of the
reference: weights are not stored in the fixtures but regenerated from a
recorded recipe (numpy default_rng(seed), discard ``skip`` normals, then
``normal(0, 0.02)`` per shape in order, +1 for 1-D ``*weight`` tensors).
"""

from __future__ import annotations

import ast
import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def seeded_parameters(recipe: dict) -> dict[str, np.ndarray]:
    rng = np.random.default_rng(int(recipe["seed"]))
    rng.normal(size=int(recipe["skip"]))
    out: dict[str, np.ndarray] = {}
    for name, shape in recipe["shapes"]:
        value = rng.normal(0, 0.02, tuple(shape)).astype(np.float32)
        if value.ndim == 1 and name.endswith("weight"):
            value += np.float32(1)
        out[name] = value
    return out


def load_fixture(name: str) -> dict[str, np.ndarray]:
    """Arrays of ``tests/golden/<name>`` plus weights regenerated from its recipe."""
    with np.load(GOLDEN / name, allow_pickle=False) as archive:
        arrays = {k: np.array(archive[k]) for k in archive.files}
    if "metadata" in arrays:
        meta = json.loads(str(arrays["metadata"]))
        # some recordings store nested fields as Python literals (data only)
        meta = {k: (ast.literal_eval(v) if isinstance(v, str) and v[:1] in "{[" else v) for k, v in meta.items()}
        arrays["__metadata__"] = meta  # type: ignore[assignment]
        recipe = meta.get("weight_recipe")
        if recipe is not None:
            arrays.update(seeded_parameters(recipe))
    return arrays


def load_boundary(name: str) -> tuple[dict, dict[str, np.ndarray]]:
    """A ``maisi/<name>.{json,npz}`` boundary: manifest and arrays (+ recipe weights)."""
    manifest = json.loads((GOLDEN / "maisi" / f"{name}.json").read_text())
    with np.load(GOLDEN / "maisi" / f"{name}.npz", allow_pickle=False) as archive:
        arrays = {k: np.array(archive[k]) for k in archive.files}
    if "weight_recipe" in manifest:
        arrays.update(seeded_parameters(manifest["weight_recipe"]))
    return manifest, arrays
