"""Writes route_literal.json: the routing known answer the reference's own test
states (tests/test_moelan.py:64-72 of moelan), as data. The values are typed in
here from that test; nothing of the reference is imported or run."""
import json
from pathlib import Path

data = {
    "source": "moelan tests/test_moelan.py:64-72",
    "logits": [[0.0, 3.0, 1.0, 2.0], [5.0, 0.0, 0.0, 4.0]],
    "top_k": 2,
    "normalize": True,
    "idx": [[1, 3], [0, 3]],
    "experts": [0, 1, 3],
    "rows_of_expert_3": [0, 1],
}
(Path(__file__).parent / "route_literal.json").write_text(json.dumps(data, indent=1) + "\n")
