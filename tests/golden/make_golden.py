"""Writes golden_vectors.json: known-answer vectors transcribed from the
reference's own tests (values are literals in those files; nothing of the
reference is imported or run).

  contract_audit    docs/test_contract_audit.py:8-46 (S=3, H=2, M=2, all six graft ops)
  down_orientation  tests/down_orientation_roundtrip.cpp:63-77,116,141-200 and
                    tests/test4_down_checkpoint_roundtrip.cpp:49-53,148
  contract_probe    src/graft_ops_impl.inc:158-212 (one-hot contract probe)
  bake_sentinel     tests/test22_shadow_bake_sentinel.cpp:72-99
  test6_f32         tests/test6_stack_vs_bake_f32.cpp:36-58,199-205
"""
import json
import os

G = {
    "contract_audit": {
        "S": 3, "H": 2, "M": 2,
        "x_h": [[1.0, 2.0], [3.0, 4.0]],
        "x_i": [[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]],
        "dy_s": [[1.0, 0.0, 0.0], [0.0, 2.0, 1.0]],
        "dx_h": [[1.0, 0.0], [0.5, 2.0]],
        "delta_exp": [[0.5, 0.0], [0.0, 1.0], [0.25, 0.0]],
        "delta_ctr_math": [[0.5, 0.0, 0.25], [0.0, 1.0, 0.0]],
        "expected": {
            "expand_fwd": [[0.5, 2.0, 0.25], [1.5, 4.0, 0.75]],
            "expand_wgrad": [[1.0, 2.0], [6.0, 8.0], [3.0, 4.0]],
            "expand_igrad": [[0.5, 0.0], [0.25, 2.0]],
            "contract_fwd": [[1.25, 2.0], [3.5, 5.0]],
            "contract_wgrad_math": [[3.0, 4.5, 6.0], [8.0, 10.0, 12.0]],
            "contract_wgrad_storage": [[3.0, 8.0], [4.5, 10.0], [6.0, 12.0]],
            "contract_igrad": [[0.5, 0.0, 0.25], [0.25, 2.0, 0.125]],
        },
    },
    "down_orientation": {
        "S": 3, "H": 2, "M": 2, "input_stride": 6,
        "w_storage": [[0.5, 0.0], [0.0, 1.0], [0.25, 0.0]],
        "x": [[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]],
        "dy": [[1.0, 0.0], [0.5, 2.0]],
        "expected_forward": [1.25, 2.0, 3.5, 5.0],
        "expected_wgrad_storage": [3.0, 8.0, 4.5, 10.0, 6.0, 12.0],
    },
    "contract_probe": {
        "M": 2, "S": 64, "H": 64, "input_stride": 128,
        "input": [[0, 3, 2.0], [1, 17, -5.0]],
        "weight": [[3, 11, 7.0], [17, 23, -13.0], [29, 31, 19.0]],
        "expected_nonzero": [[0, 11, 14.0], [1, 23, 65.0]],
    },
    "bake_sentinel": {
        "S": 3, "H": 513, "layers": 2,
        "value": "(l*100 + p*10 + s)*1000 + h + 1",
        "tol_abs": 0.5, "tol_rel": 0.005,
    },
    "test6_f32": {
        "S": 3, "H": 2, "D": 4, "F": 6, "M": 2,
        "gate0": "(i+1)*0.1", "up0": "(i+1)*0.07", "down0": "(i+1)*0.05", "x": [1, 2, 3, 4, 5, 6, 7, 8],
        "deltas": {"g0": [0.5, 0.1], "g1": [0.3, 0.2], "u0": [0.9, 0.15], "u1": [0.7, 0.05],
                   "d0": [1.2, 0.08], "d1": [1.0, 0.12]},
        "delta_rule": "v[i*H+j] = b + i*step + j",
        "tol_abs": 1e-4, "tol_rel": 1e-6,
    },
}

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden_vectors.json")
    with open(out, "w") as f:
        json.dump(G, f, indent=1)
    print("wrote", out)
