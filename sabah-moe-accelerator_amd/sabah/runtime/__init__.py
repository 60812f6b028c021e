"""Host harness of the MUL_MAT_ID expert path: ctypes binding (rt), HBM bank,
executor, routing and workload definitions."""
