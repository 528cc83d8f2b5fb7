"""CPU oracle for the Gemma 4 E2B attention path -- test infrastructure only.

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg. The product package slang_amd/ never imports it.
"""
from .attention import *  # noqa: F401,F403
