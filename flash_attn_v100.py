"""Drop-in module name of the reference extension (``import flash_attn_v100``).

Re-exports the MI355X implementation in ``flash_attn_v100_amd`` under the
reference's function names and positional signatures (flash_attn.cpp:224-255).
"""
from flash_attn_v100_amd import *  # noqa: F401,F403
from flash_attn_v100_amd import API_NAMES as _API_NAMES

__all__ = list(_API_NAMES)
