"""CPU oracle for TriangleMix paged sparse prefill attention.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (the HIP library, the
torch adapter, the ``trianglemix`` Python package) imports, links or calls
anything under ``oracle/``.  The only permitted callers are ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``, and
there only as the checker or the timed CPU baseline, never as the thing that
is measured or shipped.

Modules:

* ``geometry``  -- integer restatement of the reference's mask, span, interval,
  page-address and work-accounting rules (pure Python).
* ``cache``     -- the paged KV write upstream of the attention (slot of a
  logical token, scatter of a chunk's K/V rows into their pages).
* ``attention`` -- floating-point restatement of the reference's masked paged
  GQA attention: a float64 numpy version for small cases and a float32
  PyTorch CPU version (the reference's own oracle method) for larger ones.

Each function cites the reference file:line it restates.  How every function
is pinned (reference known-answer tests, closed forms, brute force, library
routines) is listed in the header of each module.
"""
