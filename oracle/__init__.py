"""ORACLE -- test infrastructure, not product. The CPU restatement of the reference Loopback read that checks the
HIP path. Importable only from tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg."""
