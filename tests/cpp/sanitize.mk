# Host AddressSanitizer + UndefinedBehaviorSanitizer build of the host C++
# (the reference builds its runtime, backends and C++ tests the same way,
# CMakeLists.txt:51-69). Run by tests/test_host_sanitizers.py on the CPU box:
#
#   make -f tests/cpp/sanitize.mk OUT=<dir> -j8
#
# Sanitized: the core (core/*.cpp), HipBackend (hip_backend.cpp), the C ABI's
# runtime layer (runtime.hip: pool, streams, copies, events; host code only is
# instrumented), the CPU oracle, and the C++ tests. The gfx950 kernel objects
# (tensor.cx_amd/_build/*.o from the regular build) are linked in unchanged:
# nothing launches them without a device.
#
# Everything is compiled by the ROCm clang so that one sanitizer runtime is
# linked; the HIP source takes the flags through -Xarch_host.

ROOT := $(abspath $(dir $(lastword $(MAKEFILE_LIST)))/../..)
OUT ?= $(ROOT)/tests/cpp/_san
ROCM ?= /opt/rocm
CXX := $(ROCM)/llvm/bin/clang++
HIPCC := $(ROCM)/bin/hipcc
PKG := $(ROOT)/tensor.cx_amd
BUILD := $(PKG)/_build

SAN := -fsanitize=address,undefined -fno-sanitize-recover=undefined -fno-omit-frame-pointer
CXXFLAGS := -std=c++20 -O1 -g -ffp-contract=off -Wall -Wno-unused-result $(SAN) \
            -I$(PKG)/cpp -I$(ROOT)/include -I$(PKG)/csrc
HIPFLAGS := --offload-arch=gfx950 -std=c++20 -O1 -g -fPIC -ffp-contract=off \
            -Xclang -target-feature -Xclang -packed-fp32-ops \
            -Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined \
            -Xarch_host -fno-sanitize-recover=undefined -Xarch_host -fno-omit-frame-pointer \
            -I$(ROOT)/include -I$(PKG)/csrc
LDFLAGS := $(SAN) -pthread -L$(ROCM)/lib -Wl,-rpath,$(ROCM)/lib

CORE_SRCS := $(wildcard $(PKG)/cpp/tensorcx/core/*.cpp)
CORE_OBJS := $(patsubst $(PKG)/cpp/tensorcx/core/%.cpp,$(OUT)/core_%.o,$(CORE_SRCS))
KERNEL_OBJS := $(filter-out $(BUILD)/runtime.o,$(wildcard $(BUILD)/*.o))
KERNEL_OBJS := $(filter-out $(BUILD)/cxx_%,$(KERNEL_OBJS))

TESTS := $(OUT)/pool_host_test $(OUT)/oracle_kat_test $(OUT)/device_interval_test \
         $(OUT)/launch_grid_test $(OUT)/hip_backend_contract

.PHONY: all
all: $(TESTS)

$(OUT):
	mkdir -p $(OUT)

$(OUT)/runtime.o: $(PKG)/csrc/runtime.hip | $(OUT)
	$(HIPCC) $(HIPFLAGS) -c $< -o $@

$(OUT)/core_%.o: $(PKG)/cpp/tensorcx/core/%.cpp | $(OUT)
	$(CXX) $(CXXFLAGS) -c $< -o $@

$(OUT)/hip_backend.o: $(PKG)/cpp/tensorcx/backends/hip/hip_backend.cpp | $(OUT)
	$(CXX) $(CXXFLAGS) -c $< -o $@

$(OUT)/%.o: $(ROOT)/tests/cpp/%.cpp | $(OUT)
	$(CXX) $(CXXFLAGS) -c $< -o $@

$(OUT)/oracle.o: $(ROOT)/oracle/oracle.cpp | $(OUT)
	$(CXX) $(CXXFLAGS) -c $< -o $@

$(OUT)/pool_host_test: $(OUT)/pool_host_test.o $(OUT)/runtime.o
	$(CXX) -o $@ $^ $(LDFLAGS) -lamdhip64

$(OUT)/oracle_kat_test: $(OUT)/oracle_kat_test.o $(OUT)/oracle.o
	$(CXX) -o $@ $^ $(LDFLAGS)

$(OUT)/device_interval_test: $(OUT)/device_interval_test.o $(OUT)/core_profiling.o
	$(CXX) -o $@ $^ $(LDFLAGS)

$(OUT)/launch_grid_test: $(OUT)/launch_grid_test.o
	$(CXX) -o $@ $^ $(LDFLAGS)

$(OUT)/hip_backend_contract: $(OUT)/hip_backend_contract.o $(OUT)/hip_backend.o $(CORE_OBJS) \
                             $(OUT)/runtime.o $(KERNEL_OBJS)
	$(CXX) -o $@ $^ $(LDFLAGS) -lamdhip64

# The compile and link line, for a test that plants a mistake in a program of
# its own to show that the sanitizers report it.
.PHONY: print-cxx
print-cxx:
	@echo $(CXX) $(CXXFLAGS) $(LDFLAGS)
