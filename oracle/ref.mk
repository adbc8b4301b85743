# Builds the reference's own phase0 CPU twin (the C++ restatement of its CUDA kernels) from
# the sources where they lie in the reference tree, plus the C entry points of ref_shim.cpp,
# into oracle/_ref/ (git-ignored). Test infrastructure only. The flags are those the
# reference builds its CPU extension with (phase0/splat2d/ops.py:39: -O2 -Wall -Werror),
# without -Werror since the shim is ours.
REF ?= /root/reference/phase0/csrc/macrotile
CXX ?= g++
OUT = _ref/libsplat2d_ref.so

all: $(OUT)

$(OUT): ref_shim.cpp $(REF)/splat2d_cpu.cpp $(REF)/splat2d_common.h
	mkdir -p _ref
	$(CXX) -O2 -Wall -std=c++17 -fPIC -shared -I$(REF) $(REF)/splat2d_cpu.cpp ref_shim.cpp -o $@

clean:
	rm -f $(OUT)

.PHONY: all clean
