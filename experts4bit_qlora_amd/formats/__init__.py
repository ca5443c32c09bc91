"""On-disk expert formats read by the fast path (MXFP4)."""
