"""Test infrastructure only: the CPU restatement of the reference encoder forward.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or the timed CPU
baseline).  The product (``tiktoktechjam2026track3_amd``) never imports it.
"""

from .encoder_oracle import (  # noqa: F401
    ORACLE_ATTENTION_BLOCK_ROWS,
    attention_rows,
    compare,
    encoder_forward,
    encoder_forward_sequences,
    encoder_layer,
    final_norm,
    generate_case,
    init_state_dict,
    pack_qkv,
)
