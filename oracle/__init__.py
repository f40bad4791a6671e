"""CPU oracle for the packed varlen causal GQA attention path: test infrastructure only.

Imported by `tests/`, `__graft_entry__.smoke()` and `bench.py`'s cpu_baseline leg, as the checker.
The product package `hackaton_amd` never imports it.
"""
