"""CPU oracle for the CacheSlide reuse-attention hot path -- TEST INFRASTRUCTURE ONLY.

numpy (and stdlib ``math.fsum``) restatements of the reference algorithms, each
function citing the reference file:line it follows (paths relative to the
CacheSlide repository).  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or the timed CPU baseline; the product (``cacheslide_amd``) never
imports it.

Modules:
  ccpe   -- CoPE positions, interpolated bias, cope_attention, path validation,
            the two attention policies (position.py, attention.py)
  wca    -- WCA deviation/weights/cosine/state and the fp64 blend (wca.py)
  slide  -- paged-slot scatter/gather, relocation, free-slot order
            (paged.py, slide.py)
  rows   -- the selective prefill's row bookkeeping (runtime.py)

The layer snapshot pages (runtime.py:192-256) have no restatement here: their
codec is the reference's own dependency, safetensors==0.8.0
(constraints/cpu-tests.txt:4), which is installed and is itself the checker
(tests/test_snapshot_host.py); the page store's file format is pinned by known
answers (sha256 of known payloads, hand-written page files) in
tests/test_storage_host.py.

Pinning: every function is checked in tests/test_oracle.py against the
reference's own closed-form test vectors (tests/test_position.py,
test_attention_policies.py, test_wca.py, test_slide.py, test_paged.py), against
brute force on tiny inputs and against library reductions (E = 0 reduces CCPE
to causal softmax attention; saturated rows reduce it to attention plus a
per-row constant).
"""
