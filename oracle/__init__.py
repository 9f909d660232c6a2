"""CPU oracle for the NF4 quantized-linear path (test infrastructure only; see nf4_oracle)."""
from .nf4_oracle import *  # noqa: F401,F403
