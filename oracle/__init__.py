"""The CPU oracle (test infrastructure). Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg import this package, and only as the checker."""

from .binding import Oracle, OracleSession, build_oracle, load_oracle, tensors_in_order  # noqa: F401
