"""`import enceladus` for drop-in user code: an alias of the MI355X backend package.

Existing kernels keep `import enceladus` and `import enceladus.language as tl`; both names
resolve to `enceladus_amd` and its modules (one module object each, so `isinstance` and
identity checks agree).
"""

import sys

import enceladus_amd as _pkg
from enceladus_amd import language as _language

sys.modules[__name__] = _pkg
sys.modules[__name__ + ".language"] = _language
