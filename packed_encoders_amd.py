"""Importable alias of the package directory ``packed-encoders_amd/``.

A hyphen cannot appear in an ``import`` statement, so this module imports the directory by
name and registers it, and every submodule it has loaded, under ``packed_encoders_amd``:
``import packed_encoders_amd as pe`` and ``from packed_encoders_amd import forward`` then
return the very same module objects (no second copy, no duplicated state).
"""

import importlib
import sys

_NAME = "packed-encoders_amd"
_package = importlib.import_module(_NAME)
for _key, _module in list(sys.modules.items()):
    if _key == _NAME or _key.startswith(_NAME + "."):
        sys.modules["packed_encoders_amd" + _key[len(_NAME):]] = _module
sys.modules[__name__] = _package
