# Builds libmbhip.so (gfx950 HIP kernels + the C ABI in include/mbhip.h) and
# the C restatement of the oracle.  Replaces the reference's per-kernel
# .metal -> .air -> .metallib rules (reference Makefile:37-57): one shared
# library holds every kernel, looked up by its registry `metal_function`.
#
#   make            build everything
#   make -B -j8     force a rebuild (what __graft_entry__.build() runs)
#   make test       CPU test suite

HIPCC     ?= /opt/rocm/bin/hipcc
ARCH      ?= gfx950
# Packed-fp32 VALU ops stay disabled: hipcc would otherwise form them from
# float2 code, and they are not used anywhere in this library.
HIPFLAGS  ?= -O3 -std=c++17 -fPIC --offload-arch=$(ARCH) -Wall -Wno-unused-function \
             -Xclang -target-feature -Xclang -packed-fp32-ops
CC        ?= gcc
CFLAGS    ?= -O2 -fPIC -std=c11 -Wall

SRC_DIR   := metalbench_amd/csrc
OBJ_DIR   := build/obj
LIB       := metalbench_amd/lib/libmbhip.so
HIP_SRCS  := $(wildcard $(SRC_DIR)/*.hip) $(SRC_DIR)/runtime.cpp
HIP_OBJS  := $(patsubst $(SRC_DIR)/%,$(OBJ_DIR)/%.o,$(HIP_SRCS))
HEADERS   := $(SRC_DIR)/common.h include/mbhip.h

ORACLE_LIB := oracle/lib/liboracle.so
ORACLE_SRC := $(wildcard oracle/*.c)

.PHONY: all lib oracle test clean

all: lib oracle

lib: $(LIB)

$(OBJ_DIR)/%.hip.o: $(SRC_DIR)/%.hip $(HEADERS)
	@mkdir -p $(OBJ_DIR)
	$(HIPCC) $(HIPFLAGS) -c $< -o $@

# decoder.hip: the skinny GEMM's 12 leading scalar and pointer arguments are
# preloaded into SGPRs (its other kernels start with a struct argument, which
# is not preloaded).
$(OBJ_DIR)/decoder.hip.o: HIPFLAGS += -mllvm -amdgpu-kernarg-preload-count=12

# Per-kernel register/LDS table of the kernels above, read from their own code
# objects, compiled into runtime.cpp (mb_kernel_attrs_get).
KERNEL_OBJS := $(filter-out $(OBJ_DIR)/runtime.cpp.o,$(HIP_OBJS))
RESOURCES   := build/kernel_resources.inc

$(RESOURCES): $(KERNEL_OBJS) metalbench_amd/kernel_resources.py
	python3 metalbench_amd/kernel_resources.py $(KERNEL_OBJS) > $@.tmp
	mv -f $@.tmp $@

$(OBJ_DIR)/runtime.cpp.o: $(SRC_DIR)/runtime.cpp $(HEADERS) $(RESOURCES)
	@mkdir -p $(OBJ_DIR)
	$(HIPCC) $(HIPFLAGS) -Ibuild -x hip -c $< -o $@

$(LIB): $(HIP_OBJS)
	@mkdir -p $(dir $@)
	$(HIPCC) -shared -fPIC --offload-arch=$(ARCH) --hip-link -o $@.tmp $^
	mv -f $@.tmp $@

oracle: $(ORACLE_LIB)

$(ORACLE_LIB): $(ORACLE_SRC)
	@mkdir -p $(dir $@)
	$(if $(ORACLE_SRC),$(CC) $(CFLAGS) -shared -o $@ $(ORACLE_SRC) -lm,@true)

test:
	python -m pytest tests -x -q -m "not gpu"

clean:
	rm -rf build $(LIB) $(ORACLE_LIB)
