"""CPU oracle for the torch-helion MI355X backend -- TEST INFRASTRUCTURE ONLY.

A plain restatement of the reference's algorithms for this path, used as the
checker: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it. The product (``torch-helion_amd/``) never
imports, calls or links anything here.

Modules and the reference code each follows:

* ``llama``     functional Llama block forward from a state dict
                (reference models/llama_block.py:28-159; causal mask and
                grouped KV heads are the configs' extensions).
* ``mamba``     functional Mamba-2 block / backbone forward, chunked scan and
                the O(S) recurrence (reference models/mamba.py:143-391,
                tests/test_mamba.py:27-38).
* ``interpret`` OpIR interpreter (reference codegen/interpret.py:18-77 with
                the op semantics of optimizer/evaluate.py:36-147).

Every function computes in float64 unless a caller asks otherwise.
Pinning (what checks each function against something independent) is listed
in tests/test_oracle.py; a function without such a check is marked
"parity unpinned" in its docstring.
"""
