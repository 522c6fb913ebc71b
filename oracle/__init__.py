"""ORACLE package — test infrastructure only.

Holds the C99 restatement of the reference CPU path (oracle.c), its ctypes
bindings (oracle.py), the GGUF writer used to build synthetic reference models
(gguf_writer.py) and the bindings to the reference compiled from its own
sources (ref.py, oracle/_ref/).  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import anything here, and only as the checker.
"""
