# oracle/_ref/libmp_ref.so: the reference's own MiniPrefix CPU path (engine,
# scheduler, KV manager, prefix cache, CpuRunner and the TinyInfer core it
# uses), compiled directly from its sources under $(REF) -- never copied --
# with the reference's default flags (no -march, so SSE2 without FMA),
# plus this repository's C entry points and oracle glue. Only where the
# reference tree exists; the product never links it.
REF ?= /root/reference
REPO := $(abspath $(HERE)..)
REF_OUT := $(HERE)_ref
REF_SOURCES = $(wildcard $(REF)/src/core/*.cpp) $(wildcard $(REF)/src/core/memory/*.cpp) \
	$(REF)/src/backend/cpu/matmul_kernel.cpp $(REF)/src/backend/cpu/gemm_epilogue.cpp \
	$(wildcard $(REF)/src/ops/*.cpp) \
	$(wildcard $(REF)/miniprefix/src/kv/*.cpp) $(REF)/miniprefix/src/scheduler/scheduler.cpp \
	$(REF)/miniprefix/src/engine/engine.cpp $(REF)/miniprefix/src/model/model.cpp \
	$(REF)/miniprefix/src/backend/cpu/llama_runner.cpp
REF_INCLUDES = -I$(REF)/miniprefix/include -I$(REF)/include -I$(REF)/src -I$(REPO)/include \
	-I$(REPO)/tinyinfer_amd/csrc/host -I$(HERE)
REF_CXXFLAGS = -std=c++17 -O2 -fPIC -w

ref:
	@if [ -d "$(REF)/miniprefix" ]; then $(MAKE) -f $(firstword $(MAKEFILE_LIST)) $(REF_OUT)/libmp_ref.so; \
	else echo "reference tree $(REF) absent: oracle/_ref not built"; fi

$(REF_OUT)/libmp_ref.so: $(HERE)ref_harness_backend.cpp $(HERE)mp_oracle.c $(HERE)mp_oracle.h \
		$(REPO)/tinyinfer_amd/csrc/host/capi.cpp $(REPO)/tinyinfer_amd/csrc/host/harness_backend.h
	mkdir -p $(REF_OUT)
	$(CC) $(CFLAGS) -c -o $(REF_OUT)/mp_oracle.o $(HERE)mp_oracle.c
	$(CXX) $(REF_CXXFLAGS) $(REF_INCLUDES) -shared -o $@ $(REF_SOURCES) $(HERE)ref_harness_backend.cpp \
		$(REPO)/tinyinfer_amd/csrc/host/capi.cpp $(REF_OUT)/mp_oracle.o -lm
