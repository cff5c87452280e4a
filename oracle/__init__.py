"""The oracle of the tile path: CPU restatements of krn's Python emulator and CPU clang backend.

TEST INFRASTRUCTURE ONLY. Only `tests/`, `__graft_entry__.smoke()` and the CPU-baseline leg of `bench.py` may
import, call, link or run anything under `oracle/`, and only as the checker: the product (`krn_amd`) never does.

Parity pins (each checked in tests/test_oracle.py):
- numerics.bf16_round: closed form on hand-picked words (ties, carries into the exponent, NaN quieting) and against
  a float64 nearest-even search over all bf16 neighbours.
- numerics.e4m3_*: the 256-entry decode formula, every finite code round-trips, and the vectorized encoder equals the
  exact rational nearest-even search on special values, midpoints and random values.
- numerics.fma32: against exact rational arithmetic (fractions) on random and adversarial triples.
- emulate / cbackend: bit-identical to each other on f32 products (the reference's own C1 claim, both being one
  fused multiply-add per k in k order), within the forward-error bound of float64 numpy on f16/bf16 GEMMs, and
  against a float64 softmax for flash attention.
"""
