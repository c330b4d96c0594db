"""MI355X counterpart of the reference's `sfu_repro` package: the activation
patch layer over the `spline_ops` HIP extension (src/sfu_repro/)."""
