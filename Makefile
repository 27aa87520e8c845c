# Top-level targets of the reference's Makefile (Makefile:8-24 there): build, the CPU
# tests, the GPU tests and one benchmark line. The build itself is sffft_amd/Makefile
# (gfx950 kernels, the C-ABI library, the `sffft` driver, the rocFFT comparator and the
# race-check build) and sffft_amd/torch.mk (the PyTorch operators).
PYTHON ?= python3

.PHONY: all sffft test test-gpu bench clean

all:
	$(MAKE) -C sffft_amd
	$(MAKE) -C sffft_amd -f torch.mk

# the `sffft` driver (the reference's default target)
sffft:
	$(MAKE) -C sffft_amd sffft

# CPU suite: oracle against the reference's golden values, selector against the
# reference's own header, C-ABI exports and argument errors, CLI argument handling
test: all
	$(PYTHON) -m pytest tests -q -m "not gpu"

# GPU suite on an MI355X: parity of every plan against the fp64 oracle, the CLI smoke
# checks of tests/precision_smoke.sh, reference pins, race-check build
test-gpu: all
	$(PYTHON) -m pytest tests -q -m gpu

# one benchmark line (JSON): B=8, H=768, L=1024 fp32 and the sweep over L = 128..8192
bench: all
	$(PYTHON) bench.py

clean:
	$(MAKE) -C sffft_amd clean
	$(MAKE) -C sffft_amd -f torch.mk clean
