"""Extract the checkpoint-contract fixtures from the reference's artifact
records (data files only; nothing of the reference is imported or run).

  rtn_v4_contract.json     the safetensors metadata and tensor inventory the
                           reference recorded for its W4G64 RTN-v4 export
                           (artifacts/qwen2-1.5b-w4g64-rtn-v4/manifest.json)
                           and the [out, in] shape of each of its 196 linear
                           layers (.../quantization-report.json)
  awq_canonical_v6_manifest.json
                           the frozen AWQ v6 manifest, verbatim
                           (artifacts/qwen2-1.5b-w4g64-awq-canonical-v6/manifest.json)

Run from the repository root: python tests/golden/make_checkpoint_fixtures.py
"""

import json
import shutil
from pathlib import Path

REFERENCE = Path("/root/reference/artifacts")
HERE = Path(__file__).resolve().parent


def main() -> None:
    manifest = json.loads((REFERENCE / "qwen2-1.5b-w4g64-rtn-v4/manifest.json").read_text())
    report = json.loads((REFERENCE / "qwen2-1.5b-w4g64-rtn-v4/quantization-report.json").read_text())
    fixture = {
        "safetensors_metadata": manifest["artifact"]["safetensors_metadata"],
        "tensor_inventory": manifest["artifact"]["tensor_inventory"],
        "num_linear_layers": report["num_linear_layers"],
        "linear_shapes": {name: layer["shape"] for name, layer in report["layers"].items()},
    }
    (HERE / "rtn_v4_contract.json").write_text(json.dumps(fixture, indent=1, sort_keys=True) + "\n")
    shutil.copyfile(REFERENCE / "qwen2-1.5b-w4g64-awq-canonical-v6/manifest.json",
                    HERE / "awq_canonical_v6_manifest.json")


if __name__ == "__main__":
    main()
