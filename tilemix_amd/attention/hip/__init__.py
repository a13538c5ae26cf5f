"""Host launch layer over libtilemix_hip.so (replaces the reference's attention/triton/)."""
