# Builds the genuine reference engine's CPU path (no CUDA, no NCCL) straight
# from its sources under /root/reference into oracle/_ref/, plus the thin
# extern "C" shim in oracle/ref_shim.cpp. Test infrastructure only: the
# result is the checker that writes tests/golden fixtures and pins the
# restated oracle. It is never on the product path.
#
#   make -f oracle/ref.mk -j8            (from the repo root)
#
# Flags follow the reference build (CMakeLists.txt:5-7,44,57-60,123-129):
# C++20, -O3, OpenMP, no -march=native.
REF      ?= /root/reference
OUT      := oracle/_ref
CXX      ?= g++
CXXFLAGS := -std=c++20 -O3 -fPIC -fopenmp -DGAI_OPENMP=1 -I$(REF) -w

SRCS := $(wildcard $(REF)/core/*.cpp) $(wildcard $(REF)/tokenizer/*.cpp) \
        $(wildcard $(REF)/model/*.cpp) $(wildcard $(REF)/format/*.cpp) \
        $(wildcard $(REF)/training/*.cpp) $(wildcard $(REF)/inference/*.cpp) \
        $(wildcard $(REF)/quantization/*.cpp) $(wildcard $(REF)/evaluation/*.cpp)
OBJS := $(patsubst $(REF)/%.cpp,$(OUT)/obj/%.o,$(SRCS))

all: $(OUT)/libgai_ref.so

$(OUT)/obj/%.o: $(REF)/%.cpp
	@mkdir -p $(dir $@)
	$(CXX) $(CXXFLAGS) -c $< -o $@

$(OUT)/obj/ref_shim.o: oracle/ref_shim.cpp
	@mkdir -p $(dir $@)
	$(CXX) $(CXXFLAGS) -c $< -o $@

$(OUT)/libgai_ref.so: $(OBJS) $(OUT)/obj/ref_shim.o
	$(CXX) -shared -fopenmp -o $@ $^ -lpthread

clean:
	rm -rf $(OUT)

.PHONY: all clean
