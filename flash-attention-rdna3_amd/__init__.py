"""ComfyUI custom-node entry point (reference __init__.py): ComfyUI loads this
folder as a package and reads NODE_CLASS_MAPPINGS / NODE_DISPLAY_NAME_MAPPINGS.

Loaded as a package, the adapter is imported relative to this folder, so a
different ``fa_rdna3`` installed elsewhere is never picked up.  Loaded as a
plain module, this folder goes to the front of ``sys.path``; an ``fa_rdna3``
already imported from somewhere else is an error rather than a silent mix.
"""

import os
import sys

if __package__:
    from .fa_rdna3.comfyui import NODE_CLASS_MAPPINGS, NODE_DISPLAY_NAME_MAPPINGS
else:
    _here = os.path.dirname(os.path.abspath(__file__))
    _loaded = sys.modules.get("fa_rdna3")
    _loaded_file = getattr(_loaded, "__file__", None) if _loaded is not None else None
    if _loaded is not None and not (_loaded_file and os.path.abspath(_loaded_file).startswith(_here + os.sep)):
        raise RuntimeError("A different fa_rdna3 package is already loaded; restart ComfyUI "
                           "before loading this custom node")
    if _here not in sys.path:
        sys.path.insert(0, _here)
    from fa_rdna3.comfyui import NODE_CLASS_MAPPINGS, NODE_DISPLAY_NAME_MAPPINGS

__all__ = ["NODE_CLASS_MAPPINGS", "NODE_DISPLAY_NAME_MAPPINGS"]
