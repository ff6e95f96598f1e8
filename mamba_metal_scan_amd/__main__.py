"""`python -m mamba_metal_scan_amd` builds the gfx950 library in place."""
from .build import build_library

if __name__ == "__main__":
    print(build_library(verbose=True))
