"""Oracle: CPU restatement of Knowledgator/PolyLoRA's LoRA path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` import this package, and only for
expected values (or, in ``bench.py``, as the timed CPU baseline).  The product package
``polylora_amd`` never imports, links or runs anything from here.

Modules (each function cites the reference file:line it restates):

* ``lora``  — the per-row fallback LoRA math (layers.py:112-134), the input
  shaping branches (layers.py:72-110), the reference-layout SGMV operator
  semantics (sgmv.py:63-138, :178-275), the right-padding rule
  (context.py:37-45) and the PEFT -> store layout (store.py:221-255).
* ``plan``  — the expected adapter-major token grouping of a forward.
* ``slots`` — the GPU slot bookkeeping (cache.py:60-162) as plain Python.
* ``model`` — a model wrapper that runs ``lora.reference_forward`` in place
  of every target nn.Linear, i.e. the reference's fallback forward.

How each part is pinned (tests/test_oracle.py): brute-force loops on tiny
inputs, the textbook LoRA closed form y = W x + b + (alpha / r) B A x,
invariants (rank-0 and padding rows bitwise base, weights beyond the rank
never read, linearity in B), planted mistakes that the checks must catch,
and the assertions of the reference's own tests.  The reference ships no
golden vectors, and every function is pinned by the checks above, so no
vectors are recorded from the reference.
"""
