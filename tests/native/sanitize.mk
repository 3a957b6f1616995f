# AddressSanitizer + UndefinedBehaviorSanitizer build of librocketnpu's host code (each
# -fsanitize= applies to the host pass only, via -Xarch_host; device code is built without
# it) and of the CPU oracle, linked with shim_check.cpp. For machines without a GPU;
# tests/test_sanitizers.py runs it:
#   make -f tests/native/sanitize.mk -j8 && _build_asan/shim_check tests/golden
HIPCC ?= /opt/rocm/bin/hipcc
CLANG ?= /opt/rocm/llvm/bin/clang
HERE  := $(dir $(abspath $(lastword $(MAKEFILE_LIST))))
REPO  := $(abspath $(HERE)../..)
OUT   := $(REPO)/_build_asan
PKG   := $(REPO)/rocket-userspace_amd
SAN   := -Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined \
         -Xarch_host -fno-sanitize-recover=undefined -Xarch_host -fno-omit-frame-pointer
FLAGS := --offload-arch=gfx950 -x hip -std=c++17 -O1 -g -fPIC -Wno-unused-command-line-argument $(SAN) \
         -I$(REPO)/include -I$(PKG)/csrc -I$(REPO)/oracle

SRCS := $(wildcard $(PKG)/csrc/*.cpp) $(wildcard $(PKG)/csrc/*.hip)
OBJS := $(patsubst $(PKG)/csrc/%,$(OUT)/%.o,$(SRCS))

all: $(OUT)/shim_check

$(OUT)/%.o: $(PKG)/csrc/% $(wildcard $(PKG)/csrc/*.h) $(wildcard $(REPO)/include/*.h)
	@mkdir -p $(OUT)
	$(HIPCC) $(FLAGS) -c $< -o $@

$(OUT)/oracle.o: $(REPO)/oracle/oracle.c $(REPO)/oracle/oracle.h
	@mkdir -p $(OUT)
	$(CLANG) -std=c11 -O1 -g -ffp-contract=off -fsanitize=address,undefined -fno-sanitize-recover=undefined \
	    -fno-omit-frame-pointer -c $< -o $@

$(OUT)/shim_check.o: $(HERE)shim_check.cpp $(wildcard $(REPO)/include/*.h)
	@mkdir -p $(OUT)
	$(HIPCC) $(FLAGS) -c $< -o $@

$(OUT)/shim_check: $(OBJS) $(OUT)/oracle.o $(OUT)/shim_check.o
	$(HIPCC) --offload-arch=gfx950 $(SAN) -o $@ $^ -lm -lpthread

clean:
	rm -rf $(OUT)

.PHONY: all clean
