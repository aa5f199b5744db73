"""CPU restatement of flaxchat's speculative-decoding path — TEST INFRASTRUCTURE.

This package is the parity oracle. Only `tests/`, `__graft_entry__.smoke()`
and `bench.py`'s `cpu_baseline` leg may import it, and only as the checker
(or, for `cpu_baseline`, as the timed CPU restatement). The product path in
`flaxchat_amd/` never imports it and fails loudly when its HIP library is
missing.

Modules:
  model     numpy fp32 per-token forward (flaxchat/engine.py:51-177,
            flaxchat/gpt.py:44-79) and KV-cache state (engine.py:382-393).
  sampling  Philox4x32-10 (Salmon et al., SC'11), top-k / probs / Gumbel-max
            sampling (engine.py:461-482) and the accept/reject step
            (engine.py:525-592), with the engine's counter assignment.
  spec      generate_speculative in two modes: `literal` (sequential verify and
            full re-prefill on rejection, engine.py:410-608) and `rollback`
            (the engine's chunked verify + length-pointer rollback state
            machine); generate_fast (engine.py:259-376) and
            generate_with_cache (engine.py:209-253).
  engine_stream  Engine.generate (engine.py:686-838): the streaming loop
            with per-row tool-use state, forced tokens and the calculator
            tool (engine.py:614-643).

Pinning (what checks each function, beyond restating the reference):
  * philox: Random123 known-answer vectors (tests/test_oracle.py).
  * rms_norm / rope / softcap: closed forms (unit RMS, rotation preserves
    norm, RoPE of position 0 is identity, |softcap| < 15).
  * attention: float64 brute force on random tiny inputs; window inclusive
    W+1 keys; chunk == sequential.
  * forward (model.OracleModel.step, full.gpt_call): logits written by the
    reference's own PyTorch port, flaxchat/torch_port/torch_gpt.py
    GELU_GPT(mlp="relu2"), on the same weights (tests/golden/
    make_torchport_golden.py, tests/test_torchport_pin.py: within 1e-5;
    planted mistakes in full.gpt_call are caught); also a torch float64
    re-implementation written independently in the test.
  * top-k: brute-force sort with explicit tie rule; probs sum to 1.
  * accept step: hand-crafted known-answer cases (full accept, mid reject,
    last-index reject quirk, q == 0 branch, zero residual mass, short round).
  * spec literal == rollback token-for-token; spec(draft == target) ==
    generate_with_cache greedy (tests/test_engine.py:136-150 of the
    reference); generate_fast greedy == generate_with_cache greedy
    (reference tests/test_engine.py:94-103); chi-square of the first
    emitted token against the target distribution.
  * engine_stream: the calculator against the reference's own test cases
    (tests/test_engine.py:153-171 of the reference) plus hand-worked
    expressions; the tool state machine against hand-worked token
    sequences (a python block, the forced output, completion); greedy
    streaming without tool tokens == generate_with_cache greedy.
"""
