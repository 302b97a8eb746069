"""Host wrappers of the libmoba_hip.so entry points."""
