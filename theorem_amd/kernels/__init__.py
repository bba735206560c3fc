"""Drop-in kernel packages (same names and call signatures as the reference's kernels/)."""
