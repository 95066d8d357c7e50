"""The archive writer lives in the package (rustyneedle_amd/cact.py)."""
from rustyneedle_amd.cact import HEADER_FIELDS, TAG, write  # noqa: F401
