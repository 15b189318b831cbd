"""Writes tests/golden/reference_vectors.json: the known answers that the
reference's own tests hold for this path, transcribed as data (inputs and
expected outputs). Sources, relative to packages/runntime/:

  quantpack_*   test/core/weights/quantPack.test.ts:17-93 — words worked out
                by hand from the layout description
  topk_*        test/core/kernels/reduce/topkSelect.gpu.test.ts:54-72 —
                tie-breaking and the −∞ start-value behaviour
  moe_shapes    test/core/kernels/matmul/moeQuantW.gpu.test.ts:134-144 and
                the route pattern / tolerance of :31-40, :100, :127

Run: python tests/golden/make_golden.py
"""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def numbered(k, n):
    """quantPack.test.ts:12-13: output-first [n, k] ints where the logical
    [k, n] weight's row r, column c holds r·n + c."""
    return [(i % k) * n + i // k for i in range(k * n)]


def main():
    int4_in = [v - 16 if v >= 8 else v for v in numbered(4, 4)]
    vectors = {
        "quantpack_int8_one_tile": {
            "ints_nk": numbered(4, 4), "k": 4, "n": 4, "bits": 8,
            "words": [0x0C080400, 0x0D090501, 0x0E0A0602, 0x0F0B0703],
        },
        "quantpack_int4_one_tile": {
            "ints_nk": int4_in, "k": 4, "n": 4, "bits": 4,
            "words": [0xD951C840, 0xFB73EA62],
        },
        "quantpack_twos_complement": [
            {"bits": b, "ints_nk": [(-1 if i % 2 else -(2 ** (b - 1))) for i in range(16)],
             "mask": (1 << b) - 1} for b in (8, 4)
        ],
        # K = N = 8: tiles in order (unit 0, k4 0), (0, 1), (1, 0), (1, 1);
        # first byte of each tile = row 0 of the chunk's first column.
        "quantpack_tile_order": {
            "ints_nk": numbered(8, 8), "k": 8, "n": 8, "bits": 8, "n_words": 16,
            "first_bytes": [0, 32, 4, 36],
        },
        "quantpack_readback_shapes": [
            {"bits": 8, "k": 8, "n": 12}, {"bits": 4, "k": 12, "n": 8}, {"bits": 4, "k": 16, "n": 16},
        ],
        "topk_ties": {
            "x": [[5, 7, 7, 5, 7, 1], [2, 2, 2, 2, 2, 2]], "k": 4,
            "ids": [[1, 2, 4, 0], [0, 1, 2, 3]],
            "weights_row1": [0.25, 0.25, 0.25, 0.25],
        },
        # The reference kernel's documented behaviour: a logit at or below its
        # −3.4e38 start value never enters, so empty slots keep id 0.
        "topk_neg_inf": {
            "x": [["-inf", "-inf", "-inf", "-inf", 1.0]], "k": 4,
            "route": [[4, 0, 0, 0, 1, 0, 0, 0]],
        },
        "topk_shapes": [[3, 4], [7, 9], [65, 32], [5, 1000]],
        "moe_shapes": [
            {"name": "one tile, one expert", "tokens": 1, "k": 4, "n": 8, "experts": 1, "groupSize": 4},
            {"name": "fewer units than a workgroup", "tokens": 3, "k": 16, "n": 24, "experts": 4, "groupSize": 8},
            {"name": "one K chunk past the lanes", "tokens": 2, "k": 132, "n": 8, "experts": 3, "groupSize": 4},
            {"name": "one group per expert", "tokens": 2, "k": 64, "n": 72, "experts": 5, "groupSize": 64},
            {"name": "more experts than slots", "tokens": 5, "k": 32, "n": 16, "experts": 8, "groupSize": 16},
        ],
        "moe_route_gates": [0.4, 0.3, 0.2, 0.1],
        "moe_tolerance": {"atol_per_k": 1e-5, "rtol": 1e-4},
        "lcg_first": {"seed": 1, "n": 3},
    }
    with open(os.path.join(HERE, "reference_vectors.json"), "w") as f:
        json.dump(vectors, f, indent=1)


if __name__ == "__main__":
    main()
