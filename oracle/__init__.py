"""TEST INFRASTRUCTURE ONLY.

CPU restatements of the reference algorithm used to check the HIP path:
tile_oracle (C, binning + tile compositing, via ctypes) and dense_reference
(Torch dense renderers and pinhole projection).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may use this package;
the product (fast-mac-gsplat_amd/) never imports it.
"""
