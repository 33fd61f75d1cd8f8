"""Re-export of the oracle-composed MLP (oracle/mlp.py) for the tests."""
from oracle.mlp import OracleMLP  # noqa: F401
