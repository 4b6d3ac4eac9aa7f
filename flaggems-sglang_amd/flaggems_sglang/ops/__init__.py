"""Operator modules; each lists its public functions in ``__all__``."""
