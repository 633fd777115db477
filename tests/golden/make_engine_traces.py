"""Write tests/golden/engine_traces.json: step-by-step traces of the
reference's own C++ engine (built from /root/reference/engine by
oracle/build_ref.py into oracle/_ref/) on the scripted workloads of
engine_driver.CONFIGS, two seeds each. Run in the development container:

    python oracle/build_ref.py && python tests/golden/make_engine_traces.py
"""

import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import build_ref  # noqa: E402
from tests.golden.engine_driver import CONFIGS, TRACES, drive  # noqa: E402

STEPS = 80
SEEDS = (7, 8)


def main():
    ref = build_ref.load()
    if ref is None:
        sys.exit("reference engine not built; run oracle/build_ref.py first")
    out = {"steps": STEPS, "generator": "reference memforge_c built from engine/src by oracle/build_ref.py"}
    for name, cfg in CONFIGS.items():
        out[name] = {str(s): drive(ref, s, **cfg, steps=STEPS) for s in SEEDS}
    TRACES.write_text(json.dumps(out, separators=(",", ":")) + "\n")
    print(f"wrote {TRACES} ({TRACES.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
