"""CPU oracle for the packed Q6_K/Q4_K expert matmul and the Q8 KV gather.

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this
package. Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it, and only to check results (or, in the bench,
as the timed CPU baseline), never as the thing that is measured or shipped.

Every function restates the algorithm of a reference file in plain NumPy and
cites the file:line it follows (paths are relative to the reference tree of
AhmadSaeedZaidi/data-synth-tpu). How each function is pinned:

==========================  ==================================================
function                    pinned by
==========================  ==================================================
gguf.dequantize_rows        gguf-py 0.19.0 frozen vectors
                            (tests/golden/gguf_py_decoder_reference.npz, a
                            data file the reference ships) for Q4_K, Q5_K,
                            Q6_K, Q8_0, F16, BF16, F32; the scalar per-position
                            Q6_K oracle below; closed-form Q5_1/IQ4_NL
                            enumerations from the reference's tests; scalar
                            per-value Q4_0/Q4_1/Q5_0 restatements of the GGML
                            block definitions with random FP16 d and m.
packed_q6.decode_reference  agreement with gguf.dequantize_rows (independent
                            formulation) and the gguf-py vectors.
packed_q6.bf16_round        exhaustive: every BF16 bin at 0x0000/0x7FFF/
                            0x8000/0x8001 low halves against torch's RNE cast.
packed_q6.fp16_bits_to_f32  exhaustive over all 63 488 finite FP16 patterns
                            against numpy's IEEE conversion.
packed_q6.soa_offsets       planes written by the reference's own pack_q6
                            (tests/golden/packed_q6_soa_reference.npz, made
                            by tests/golden/make_soa_golden.py); round trip
                            against the product packer; a plain permutation.
packed_q6.projection_ref    FP64 dot of BF16-rounded operands; closed-form
                            checks (identity-like weights, linearity in x).
numerics.sigmoid/softmax    FP64 closed form, 2-ulp budget.
routing.route               brute-force top-k on tiny inputs; renormalised
                            weights sum to 1 within BF16 rounding.
moe.expert_ffn              brute-force per-token loop (routing_validation
                            style) vs. the compacted expert loop; zero-route
                            and poisoned-expert invariants.
kv.*                        closed forms from the reference's KV tests
                            (rounded-divisor case, zero groups, clipping).
compute.q8_matmul           exact closed form on power-of-two scales and
                            integer codes (equals x . dequant(W) in FP64);
                            zero rows give exact zeros.
moe.shared_gate             closed forms (one-hot routers, sigmoid(0),
                            saturation, the BF16 rounding of the logit).
==========================  ==================================================
"""
