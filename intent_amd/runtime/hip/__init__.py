"""The hip provider's runtime: ctypes library, operator table, prepared calls."""
