"""flash_attn_interface — FA-3 argument order, resolved to fable_attn.fa3_interface."""
from fable_attn.fa3_interface import *  # noqa: F401,F403
from fable_attn.fa3_interface import get_scheduler_metadata  # noqa: F401
