# Builds libsffft_torch.so, the PyTorch operators (csrc/torch_ops.cpp): host code only, compiled
# with the host compiler against the installed torch's headers and libraries, linked to
# libsffft.so (which the main Makefile builds). Kept apart from the kernel build so that the
# kernel recipe, and so the kernel-source stamp of the profile summaries, does not depend on it.
#   make -C sffft_amd -f torch.mk
ROCM ?= /opt/rocm
PYTHON ?= python3
CXX ?= g++
TORCH_DIR := $(shell $(PYTHON) -c "import os, torch; print(os.path.dirname(torch.__file__))")
TORCH_ABI := $(shell $(PYTHON) -c "import torch; print(int(torch._C._GLIBCXX_USE_CXX11_ABI))")
# hip_runtime_api.h needs its platform named when a host compiler includes it; USE_ROCM is the
# configuration torch's own ROCm build used for these headers
TORCH_FLAGS = -O2 -std=c++17 -fPIC -D__HIP_PLATFORM_AMD__ -DUSE_ROCM -D_GLIBCXX_USE_CXX11_ABI=$(TORCH_ABI) \
	-I../include -I$(TORCH_DIR)/include -I$(TORCH_DIR)/include/torch/csrc/api/include -I$(ROCM)/include

.PHONY: all clean
all: libsffft_torch.so

libsffft_torch.so: csrc/torch_ops.cpp ../include/sffft.h libsffft.so
	$(CXX) $(TORCH_FLAGS) -shared -o $@ $< -L. -lsffft -L$(TORCH_DIR)/lib -lc10 -lc10_hip -ltorch_cpu -ltorch \
	  -Wl,-rpath,'$$ORIGIN' -Wl,-rpath,$(TORCH_DIR)/lib

clean:
	rm -f libsffft_torch.so
