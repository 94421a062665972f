"""`_batteries`: alias of the `_batmobile` extension.

The reference package imports its extension as `_batteries`
(python/batmobile/__init__.py:12) while its binding declares `_batmobile`
(python/bindings.cpp:597) and its autograd module imports `_batmobile`
(python/batmobile/autograd.py:15).  Both names resolve to the same module here.
"""
import torch  # noqa: F401  (loads the HIP runtime torch was built with)
from _batmobile import *  # noqa: F401,F403
from _batmobile import __doc__  # noqa: F401
