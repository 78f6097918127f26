"""ORACLE — test infrastructure only (CPU restatement of HOS's training path).

Importable by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg only.
"""
