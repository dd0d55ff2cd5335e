"""Package version of the MI355X KV-movement backend."""

__version__ = "0.1.0"
#: Version of the reference public KV API whose names and signatures this
#: package mirrors (musa_aiter/version.py:1 of the reference).
REFERENCE_API_VERSION = "0.5.0"
