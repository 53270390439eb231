"""Executable bundles the HIP provider loads (hand-built gfx950 code objects)."""

from tensor_amd.artifacts.hip import ArtifactError, read_artifact, validate_manifest, write_artifact

__all__ = ["ArtifactError", "read_artifact", "validate_manifest", "write_artifact"]
