"""Test infrastructure: the CPU parity oracle for the MI355X backend.

NOT product code. Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline`
leg may import it, and only as the checker. The product package (`enceladus_amd`) never
imports or calls anything here; with the HIP library missing it raises instead of
falling back to this interpreter.

`oracle.interpreter` restates the reference language's `ENCELADUS_INTERPRET=1`
interpreter from scratch (reference: src/enceladus/interpreter/interp.py and the `_i_*`
handlers in src/enceladus/language/ops.py). `oracle.reference_np` holds the examples'
NumPy closed forms (reference: examples/*.py `reference()` functions).

Pinning (what checks each function against something other than its own formula) is
listed in the interpreter module's docstring.
"""
