"""CPU oracle for the YANchor batched recurrent hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``yanchor_amd``) imports,
calls or links anything here.  The only permitted users are ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``, and
they use it strictly to check results (or as the timed CPU path), never as the
thing that is measured or shipped.

Each module restates one part of the reference's algorithm on the CPU and cites
the reference file:line it follows:

* ``oracle.gdn``      gated delta rule: recurrent step, chunked form, varlen
                      packing, the fused decode gates.
* ``oracle.anchor``   fixed-slot anchor memory: committed read with the
                      zero-logit sink, push + Top-K commit, ``select_topk`` /
                      ``merge_topk`` / ``exclusive_prefix_topk``.
* ``oracle.sampling`` counter hash, top-k/top-p counter sampler, the top-20
                      sampler, the dense presence penalty.
* ``oracle.slots``    slot bookkeeping, cu_seqlens, compaction keep-lists,
                      refill planning.
* ``oracle.glue``     the decode-layer glue: RMSNorm, gated RMSNorm, conv
                      update (torch and CUDA-backend forms), GDN gates, RoPE,
                      the memory projections, the SWA ring read and write.

Floating-point parts are written with torch on the CPU (float64 by default so
they act as the exact answer; float32 when timed as the CPU baseline).  Integer
parts use Python ints / numpy.

Pinning status of every function (closed forms, invariants, brute force, golden
vectors) is listed in the module docstrings; a function with no such check says
"parity unpinned".
"""
