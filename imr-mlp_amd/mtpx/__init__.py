"""Python front end of the MI355X MTP path: ctypes binding of libmtpx.so
(capi) and the deterministic synthetic workloads (synth)."""
