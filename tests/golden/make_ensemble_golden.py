"""Copy the reference's default inference configuration (configs/default_inference.json: the
member dictionaries of the preprocessing ensemble in front of NoriRegressor) into a fixture.

The file is configuration data -- step names and their parameters -- and the test that reads
it (tests/test_ensemble_host.py) holds nori_amd.ensemble.DEFAULT_MEMBERS to it. Only this
container holds the reference (at /root/reference).

Usage: python tests/golden/make_ensemble_golden.py   (writes tests/golden/default_inference_members.json)
"""

from __future__ import annotations

import json
import os

SOURCE = "/root/reference/src/synthefy_nori/configs/default_inference.json"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "default_inference_members.json")


def main():
    with open(SOURCE) as f:
        members = json.load(f)
    with open(OUT, "w") as f:
        json.dump(members, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"wrote {OUT}: {len(members)} members")


if __name__ == "__main__":
    main()
