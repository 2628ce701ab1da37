"""Writes known_answers.json: the known-answer vectors that the reference's
own unit tests hold for this path, as data (inputs and expected outputs).

Sources (deepsheth3/Omnistack-RS):
  tests/unit/test_quant.py:167-176   codes (5, 3) -> byte 53
  tests/unit/test_quant.py:178-182   all codes 15 -> all bytes 0xFF
  tests/unit/test_quant.py:422-441   bytes [0x53,0x24,0x71,0xA6] -> codes [3,5,4,2,1,7,6,10]
  tests/unit/test_quant.py:604-609   seed table (user_id, row_seed) -> (user_id % 1024) ^ row_seed
  tests/unit/test_hadamard.py:166-188  H4 [1,2,3,4] -> [10,-2,-4,0] / sqrt(4)
plus the C++ standard's check value for std::mt19937 ([rand.predef]: the
10000th draw of a default-seeded engine).

    python tests/golden/make_known_answers.py
"""
import json
import os

DATA = {
    "pack": [
        {"codes_prefix": [5, 3], "byte0": 53, "source": "tests/unit/test_quant.py:167-176"},
        {"codes_all": 15, "bytes_all": 255, "source": "tests/unit/test_quant.py:178-182"},
    ],
    "unpack": [
        {"bytes_prefix": [0x53, 0x24, 0x71, 0xA6], "codes_prefix": [3, 5, 4, 2, 1, 7, 6, 10],
         "source": "tests/unit/test_quant.py:422-441"},
        {"bytes_all": 255, "codes_all": 15, "source": "tests/unit/test_quant.py:416-420"},
    ],
    "seed": {"cases": [[0, 7, 7], [1, 7, 6], [1024, 7, 7], [1025, 7, 6], [5, 3, 6]],
             "fields": ["user_id", "row_seed", "seed"], "source": "tests/unit/test_quant.py:604-609"},
    "wht4": {"x": [1.0, 2.0, 3.0, 4.0], "y": [5.0, -1.0, -2.0, 0.0],
             "source": "tests/unit/test_hadamard.py:166-188"},
    "mt19937": {"seed": 5489, "draw": 10000, "value": 4123659995, "source": "C++ [rand.predef]"},
}

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answers.json")
    with open(out, "w") as f:
        json.dump(DATA, f, indent=1)
        f.write("\n")
