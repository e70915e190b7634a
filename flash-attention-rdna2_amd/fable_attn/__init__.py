"""fable_attn — exact attention for MI355X (gfx950) behind the flash_attn API.

    import fable_attn; fable_attn.install_as_flash_attn()   # `import flash_attn` now resolves here
or directly:
    from fable_attn import flash_attn_func

Kernels live in libfable_attn_hip.so (C-ABI, include/fable_attn_abi.h); this package is the
host-side mirror of the reference's Python interface (package/fable_attn/__init__.py:12-101).
"""
import sys

from .flash_attn_interface import (
    flash_attn_combine,
    flash_attn_func,
    flash_attn_kvpacked_func,
    flash_attn_qkvpacked_func,
    flash_attn_varlen_func,
    flash_attn_varlen_kvpacked_func,
    flash_attn_varlen_qkvpacked_func,
    flash_attn_with_kvcache,
)

from . import torch_op

# torch.ops.fable_attn.forward, as the reference registers at import (__init__.py:23,29)
torch_op.register()

__all__ = [
    "flash_attn_func", "flash_attn_qkvpacked_func", "flash_attn_kvpacked_func",
    "flash_attn_varlen_func", "flash_attn_varlen_qkvpacked_func",
    "flash_attn_varlen_kvpacked_func", "flash_attn_combine", "flash_attn_with_kvcache",
    "install_as_flash_attn",
]

__version__ = "0.1.0"

# Version announced when installed as flash_attn: callers gate features on the FA-2 version
# (window_size, softcap, ...), so the FA-2 surface version is reported with a local suffix
# (reference __init__.py:54).
FLASH_ATTN_API_VERSION = "2.8.3+fable.mi355x." + __version__


def install_as_flash_attn():
    """Register this package under the module names foreign code imports:
    flash_attn and flash_attn.flash_attn_interface (FA-2 order) and flash_attn_interface
    (FA-3 order). The reference also aliases pure-torch helper modules (bert_padding, layers,
    modules, ops); those are outside this library's scope and are not registered."""
    from . import fa3_interface as _fi3
    from . import flash_attn_interface as _fi
    me = sys.modules[__name__]
    me.__dict__.setdefault("_fable_own_version", __version__)
    me.__version__ = FLASH_ATTN_API_VERSION
    _fi.__version__ = FLASH_ATTN_API_VERSION
    sys.modules["flash_attn"] = me
    sys.modules["flash_attn.flash_attn_interface"] = _fi
    sys.modules["flash_attn_interface"] = _fi3
    return me
