"""Packed forward, EESD engine and its host policies (the reference's solutions/ surface)."""
