"""Packed forward, EESD engine and its host policies (the reference's solutions/ surface).
Importing the package registers the "eesd" method in thesis_amd.common.methods."""

from . import method  # noqa: F401  (registers "eesd")
