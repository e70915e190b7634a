"""flash_attn.flash_attn_interface — FA-2 argument order."""
from fable_attn import FLASH_ATTN_API_VERSION as __version__  # noqa: F401
from fable_attn.flash_attn_interface import *  # noqa: F401,F403
