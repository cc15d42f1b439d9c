"""`tilec.language` host helpers (tilec/language.py), served by tilec_amd.language."""

from tilec_amd.language import cdiv  # noqa: F401

__all__ = ["cdiv"]
