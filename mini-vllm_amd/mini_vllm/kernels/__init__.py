"""Kernel seam: ``ops`` dispatches, ``extension`` builds and binds the HIP library."""
