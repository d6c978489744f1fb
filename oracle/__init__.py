"""CPU restatement of the reference's forward evaluator.  TEST INFRASTRUCTURE ONLY.

This package checks results and is never the thing measured or shipped: only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import it.  The product
(`alpha-fly_amd/chessfly` over the HIP library) must never call into it.

Modules
-------
lightcone  numpy restatement of LightCone / _SubMatrix (chessfly/brain.py:102-173); integer, bit-exact.
forward    torch-CPU restatement of ConnectomeRNN.forward (brain.py:211-229), the float32 light-cone
           forward_io (brain.py:282-329, CPU branch), the float16 deviation path (brain.py:254-280) with
           float16 storage emulated, and FlyChessNet.forward / RunningNorm / expected_value
           (chessfly/model.py:37-58, 95-110).
brute      independent fp64 brute force for tiny graphs: dense-matrix recurrence (the closed form of
           tests/test_core.py:22-27) and breadth-first-search light cones from hop distances.  These pin
           the two restatements above.

Parity pinning status (what each restated function is checked against, in tests/test_oracle.py):
  light_cone sets and sub-matrices   brute-force BFS on tiny graphs + structural invariants   pinned
  literal recurrence                 dense fp64 closed form                                   pinned
  float32 light-cone forward_io      equality with literal[out_idx] (fp64, 1e-9)              pinned
  float16 deviation forward_io       algebraic identity in fp64 (exact) + tolerance vs fp32   pinned to tolerance;
                                     the reference's exact fp16 rounding sequence (cuSPARSE    bit level unpinned
                                     accumulation order, jiterator compute type) is unknowable here
  heads / RunningNorm / move_squares closed forms and the index definition                    pinned
"""
