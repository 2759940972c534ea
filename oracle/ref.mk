# Builds the reference CPU library from its own sources under /root/reference into
# oracle/_ref/libacfun_ref.so.  It is a test oracle and the CPU baseline only; the
# product (acfun_amd/) never links or loads it.  Per-file ISA flags follow the
# reference's CMakeLists.txt:52-91 so that its runtime dispatch picks the same paths.
#   make -f oracle/ref.mk            (from the repo root)
REF    ?= /root/reference
OUT    ?= oracle/_ref
CXX    ?= g++
BASE   := -O3 -std=gnu++17 -fPIC -fopenmp -I$(REF)/include -I$(REF)/include/acfun

SRCS := gemm gemm_ref gemm_avx2 gemm_avx512 gemm_int8 gemm_int8_avx512 gemm_bf16_avx512 \
        int8_quantize int8_quantize_avx2 int8_quantize_avx512 conv_int8_direct \
        conv_int8_direct_avx512 conv1x1_int8 conv1x1_int8_avx512 autotune winograd \
        winograd_avx2 winograd_avx512 winograd43 winograd43_avx512 layers conv_int8 \
        winograd_int8 model dw dw_avx512 group_conv group_conv_avx2 group_conv_avx512 \
        maxpool_avx2 maxpool_avx512

FL_gemm_avx2              := -mavx2 -mfma
FL_gemm_avx512            := -mavx512f -mfma
FL_gemm_int8_avx512       := -mavx512f -mfma -mavx512vnni -ffp-contract=off
FL_int8_quantize_avx512   := -mavx512f -mfma -mavx512bw
FL_int8_quantize_avx2     := -mavx2 -mfma
FL_conv_int8_direct_avx512:= -mavx512f -mfma -mavx512vnni -ffp-contract=off
FL_conv1x1_int8_avx512    := -mavx512f -mfma -mavx512vnni -ffp-contract=off
FL_gemm_bf16_avx512       := -mavx512f -mfma -mavx512bf16
FL_winograd_avx2          := -mavx2 -mfma
FL_winograd_avx512        := -mavx512f -mfma
FL_winograd43_avx512      := -mavx512f -mfma
FL_winograd_int8          := -mavx512f -mavx512bw -mavx512dq -mfma
FL_dw_avx512              := -mavx512f -mfma
FL_group_conv_avx512      := -mavx512f -mfma
FL_group_conv_avx2        := -mavx2 -mfma
FL_maxpool_avx512         := -mavx512f -mfma
FL_maxpool_avx2           := -mavx2 -mfma

OBJS := $(addprefix $(OUT)/obj/,$(addsuffix .o,$(SRCS)))

all: $(OUT)/libacfun_ref.so

$(OUT)/obj/%.o: $(REF)/src/%.cpp
	@mkdir -p $(OUT)/obj
	$(CXX) $(BASE) $(FL_$*) -c $< -o $@

$(OUT)/libacfun_ref.so: $(OBJS)
	$(CXX) -shared -fopenmp -Wl,-Bsymbolic -o $@ $(OBJS)

clean:
	rm -rf $(OUT)

.PHONY: all clean
