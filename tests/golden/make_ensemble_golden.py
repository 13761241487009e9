"""Write the SHA-256 digest of the reference's default inference configuration
(configs/default_inference.json: the member dictionaries of the preprocessing ensemble in front
of NoriRegressor) as a fixture.

Only the digest of the configuration's canonical JSON form (``json.dumps(members,
sort_keys=True)``) is stored, with the member count; the test that reads it
(tests/test_ensemble_host.py) holds the digest of nori_amd.ensemble.DEFAULT_MEMBERS, in the same
canonical form, to it. Only this container holds the reference (at /root/reference).

Usage: python tests/golden/make_ensemble_golden.py   (writes tests/golden/default_inference_digest.json)
"""

from __future__ import annotations

import hashlib
import json
import os

SOURCE = "/root/reference/src/synthefy_nori/configs/default_inference.json"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "default_inference_digest.json")


def canonical_digest(members) -> str:
    return hashlib.sha256(json.dumps(members, sort_keys=True).encode()).hexdigest()


def main():
    with open(SOURCE) as f:
        members = json.load(f)
    with open(OUT, "w") as f:
        json.dump({"members": len(members), "sha256": canonical_digest(members)}, f, indent=1)
        f.write("\n")
    print(f"wrote {OUT}: {len(members)} members")


if __name__ == "__main__":
    main()
