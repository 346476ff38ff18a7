"""yanchor_amd: MI355X-native kernels for YANchor's batched recurrent hot path.

Modules mirror the reference's call sites:

* ``yanchor_amd.gdn``                 gated delta rule (decode state update, chunked
                                      varlen prefill)
* ``yanchor_amd.independent_memory``  anchor memory read / commit
* ``yanchor_amd.inference_kernels``   counter sampling, presence penalty, slot
                                      bookkeeping, packing and compaction

All compute runs in hand-written HIP kernels from ``lib/libyanchor_amd.so``
(built by ``python -m yanchor_amd.build``); there is no CPU fallback.
"""
__version__ = "0.1.0"
