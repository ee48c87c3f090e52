"""Record format, calibration and codec tables (reference: fragpack/compression)."""
