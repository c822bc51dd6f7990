"""Training drivers of the DelRec experiments that run on this package's layers."""
