"""Copy the reference's recorded golden fixtures for this path into tests/golden/.

The fixtures are data (seeded inputs and Torch-CPU / MONAI outputs recorded by
the reference project on darwin-arm64, Apache-2.0): they are copied byte for
byte, never regenerated and never executed.  Weights are not stored in them;
the reference regenerates weights from a recipe recorded in each file's
metadata (``tests/fixture_parameters.py:15-25`` of the reference), which
``tests/golden_util.py`` restates.

It also extracts the production weight inventory (tensor name, Torch shape,
on-disk layout) of the from-mask checkpoints from the reference's data file
``src/mlx_generate_ctmr/data/maisi_mlx_from_mask_weight_catalog.json`` into
``from_mask_catalog.json``.

Run once in a container that has the reference checkout:
    python tests/golden/make_golden.py /root/reference
"""

from __future__ import annotations

import json
import shutil
import sys
from pathlib import Path

FILES = (
    "source_fp32.npz",  # conv / group norm / silu / trilinear goldens
    "unet.npz",  # tiny UNet (fast path) golden + weight recipe
    "vae.npz",  # tiny VAE decode + tiled decode golden + weight recipe
    "mr.npz",  # end-to-end MR: velocity batch, 30-step latent, decoded, int16
    "mr-brain.npz",
    "rflow.npz",
    "controlnet.npz",  # tiny ControlNet weight recipe + constructor (no recorded outputs)
    "maisi/residual.json",
    "maisi/residual.npz",
    "maisi/diffusion.json",
    "maisi/diffusion.npz",
    "maisi/vae.json",
    "maisi/vae.npz",
    "maisi/scheduler.json",
    "maisi/scheduler.npz",
    "maisi/attention.json",
    "maisi/attention.npz",
    "maisi/controlnet.json",
)


def main(reference: Path) -> None:
    src_dir = reference / "tests" / "fixtures" / "darwin-arm64"
    dst_dir = Path(__file__).resolve().parent
    for name in FILES:
        dst = dst_dir / name
        dst.parent.mkdir(parents=True, exist_ok=True)
        shutil.copyfile(src_dir / name, dst)
        print(f"copied {name} ({dst.stat().st_size} bytes)")
    catalog = json.loads((reference / "src" / "mlx_generate_ctmr" / "data" /
                          "maisi_mlx_from_mask_weight_catalog.json").read_text())
    slim = {
        "source": "maisi_mlx_from_mask_weight_catalog.json (name, torch_shape, layout per tensor)",
        "networks": {
            net: [[t["name"], t["torch_shape"], t["layout"].rsplit(".", 1)[-1]] for t in spec["tensors"]]
            for net, spec in catalog["networks"].items()
        },
    }
    out = dst_dir / "from_mask_catalog.json"
    out.write_text(json.dumps(slim, separators=(",", ":")) + "\n")
    print(f"wrote {out.name} ({out.stat().st_size} bytes)")


if __name__ == "__main__":
    main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
