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
    "exact.projection_signs_exact": "tests/test_oracle_pins.py::"
                                    "test_exact_projection_signs_survive_cancellation: "
                                    "rows whose fp64 sum loses the small terms after "
                                    "+-1e30 cancellation keep the sign of the exact "
                                    "rational sum (and it equals fp64 where that is exact)",
}
