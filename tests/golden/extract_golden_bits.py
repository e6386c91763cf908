"""Extract the reference's checked-in golden bit patterns into a JSON fixture.

Source (read as text, never executed): the literal blocks between
`# --- GOLDEN BEGIN ---` and `# --- GOLDEN END ---` in the reference's
`tests/test_golden_bits.mojo` (ajhendel/mojoboost, lines 322-7660). Each
fixture (l2, logit, multi, bagged, ffrac, misscat, large) has four arrays:

  _INTS   n_trees, then per tree n_nodes and per node
          (feature, threshold_bin, left, right)
  _VALS   per-node leaf/internal values as IEEE-754 hex bits
  _RAW    per-row raw score bits (predict_raw_row / predict_raw_bins)
  _PRED   per-row response bits (predict_row / predict_proba_bins)

The fixture inputs are closed-form generators restated in
tests/golden_fixtures.py; only the expected outputs are data.

Run: python3 tests/golden/extract_golden_bits.py /root/reference/tests/test_golden_bits.mojo
"""
import json
import re
import sys
from pathlib import Path

PREFIXES = {
    "_L2": "l2",
    "_LOGIT": "logit",
    "_MULTI": "multi",
    "_BAG": "bagged",
    "_FFRAC": "ffrac",
    "_MISSCAT": "misscat",
    "_LARGE": "large",
}


def main(src: str) -> None:
    text = Path(src).read_text()
    begin = text.index("# --- GOLDEN BEGIN ---")
    end = text.index("# --- GOLDEN END ---")
    block = text[begin:end]
    out: dict = {}
    for m in re.finditer(r'comptime (\w+) = """(.*?)"""', block, re.S):
        name, body = m.group(1), m.group(2)
        prefix, kind = name.rsplit("_", 1)
        fixture = PREFIXES[prefix]
        toks = body.split()
        if kind == "INTS":
            vals = [int(t) for t in toks]
        else:
            vals = [t.lower() for t in toks]
        out.setdefault(fixture, {})[kind.lower()] = vals
    dest = Path(__file__).with_name("golden_bits.json")
    dest.write_text(json.dumps(out, separators=(",", ":")))
    print(f"wrote {dest} with fixtures {sorted(out)}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tests/test_golden_bits.mojo")
