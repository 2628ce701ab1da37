"""CPU oracle for the INT4 + QJL KV-cache codec and compressed-KV attention.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
directory; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker
(or, for ``cpu_baseline``, as the timed CPU restatement of the reference's
own CPU path).

Contents
--------
``restate``   torch (CPU, fp32) restatement of the reference's CPU code path,
              one function per reference function, each citing the reference
              file:line it follows.  Because the reference path is itself
              plain torch, the restatement uses the same torch operators in
              the same order.
``exact``     fp64 ground truth: exact QJL projections (for the sign-bit
              boundary rule), correctly rounded residual norms, brute-force
              softmax attention, explicit first-index argmin.
``mt19937``   ctypes binding of ``mt19937_ref.c``: a textbook MT19937
              (Matsumoto & Nishimura 1998) used to pin the QJL G matrix that
              the reference draws with ``torch.randint`` on a CPU generator.

How each oracle function is pinned (beyond retyping the reference) is listed
in ``PINS`` below; the tests named there fail if the restatement drifts.
"""

PINS = {
    "restate.wht": "tests/test_oracle_pins.py: H4 known answer (reference "
                   "tests/unit/test_hadamard.py:166-188), equality with the "
                   "scipy Sylvester Hadamard matrix / sqrt(128) in fp64, "
                   "self-inverse, norm preservation",
    "restate.rotate": "tests/test_oracle_pins.py::test_rotate_sign_flip_matches_"
                      "hadamard_times_flip: equals scipy's Sylvester H / sqrt(D) @ "
                      "(s * x) in fp64 at D = 128 and 32 (a flip after the transform, "
                      "or none, misses by O(1)); bf16 inputs rounded once",
    "restate.make_g_matrix": "tests/test_oracle_pins.py::test_make_g_matrix_is_one_"
                             "mt19937_stream_packed_lsb_first: every lo / hi word "
                             "equals textbook MT19937 low bits in (head, row, "
                             "column) order packed with Python integers; it is the "
                             "checker of the product's make_g_matrix "
                             "(tests/test_native_lib.py)",
    "restate.qjl_g": "tests/test_oracle_pins.py: bits equal textbook MT19937 "
                     "low bits (C, mt19937_ref.c); MT19937 itself pinned by "
                     "the C++ [rand.predef] value (10000th draw of seed 5489 "
                     "is 4123659995)",
    "restate.make_qjl_seed": "reference seed table, tests/unit/test_quant.py:604-609, 626-632",
    "restate.quantize_int4": "explicit first-index argmin loop (exact.argmin_first) "
                             "incl. ties, NaN and +-inf",
    "restate.pack_nibbles / unpack_nibbles": "reference known answers: byte 53 "
                   "(test_quant.py:167-176), 0xFF (:178-182), "
                   "[0x53,0x24,0x71,0xA6] -> [3,5,4,2,1,7,6,10] (:422-441)",
    "restate.qjl_encode_batch": "signs equal the sign of the exact fp64 "
                                "projection except where |P|/||e|| < 1e-6 "
                                "(boundary rule); all-zero residual -> 0xFF",
    "restate.quantize_heads (norms)": "within 2 ulp of the correctly rounded "
                                      "fp64 norm (exact.residual_norm)",
    "restate.dequantize_heads": "QJL estimator closed form: mean over rows of "
                                "E[(G^T b)_j] matches sqrt(2/pi)*64*e_j/||e|| "
                                "statistics; INT4+QJL MSE >= 5% below INT4 "
                                "(reference test_quant.py:308-322)",
    "restate.reference_attn": "fp64 brute-force softmax (exact.attention) at "
                              "1e-5; V=const -> const; single unmasked key -> v0",
    "restate.apply_lora_to_q": "merged-weight closed form q + x (B A)^T alpha "
                               "in fp64; sentinel -1 exactly unchanged",
    "restate.lloyd_max": "tests/test_oracle_pins.py: 16 repeated dyadic levels "
                         "are recovered exactly; max_iters=0 gives the equal-count "
                         "bin means (math.fsum, n % 16 largest left out); the "
                         "N(0,1) quantile grid converges to Max's 1960 table "
                         "(levels within 2.5e-3, MSE 0.009497)",
    "restate.qjl_reconstruct_batch": "signed sum of textbook-MT19937 G rows (an "
                                     "exact integer vector) times the fp32 scale, "
                                     "bit for bit; also via dequantize_heads",
    "restate.quantize_rows": "per-row seed (uid % 1024) ^ (base + i): codes equal "
                             "the explicit argmin, signs the exact projection signs "
                             "on each row's MT19937 G (boundary rule), norms within "
                             "2 ulp of the exact norm",
    "restate.dequantize_rows": "exact integer reconstruction with each row's own "
                               "seed, bit for bit; centroids alone without QJL",
    "restate.repeat_kv": "explicit layout known answer (kv head h on q heads "
                         "h*G .. h*G+G-1)",
    "restate.fused_attn_python": "fp64 brute force over a K / V reconstruction "
                                 "built from textbook pieces (shift unpacking, "
                                 "MT19937 G), D = 128 and 32, with and without "
                                 "QJL and the causal mask, at 2e-5",
    "restate.omni_attn_cpu": "fp64 brute force with q updated by the merged LoRA "
                             "weight (sentinel row unchanged) and scale None = "
                             "1/sqrt(128), at 2e-5",
    "exact.argmin_first / pack_bits_lsb / ulp_distance_f32 / residual_norm / "
    "projections_fp64 / exact_dot / g_from_mt / attention":
        "tests/test_oracle_pins.py::test_exact_helpers_known_answers (hand-worked "
        "cases: ties and NaN, bit order, adjacent floats, 3-4-5, exact dyadic "
        "sums, raw MT19937 low bits, uniform softmax = mean of V); g_from_mt "
        "rests on the C++ [rand.predef] MT19937 value",
    "exact.projection_signs_exact": "tests/test_oracle_pins.py::"
                                    "test_exact_projection_signs_survive_cancellation: "
                                    "rows whose fp64 sum loses the small terms after "
                                    "+-1e30 cancellation keep the sign of the exact "
                                    "rational sum (and it equals fp64 where that is exact)",
}
