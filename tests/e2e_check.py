"""The tie classification of the end-to-end tests (oracle/parity.py, the checker shared
with bench.py's parity object)."""

from oracle.parity import (classify_departures, decode, f16_bits_to_f32,  # noqa: F401
                           first_divergences, row_digests, summarise)
