# CPU-only sanitizer builds (gcc / g++, nothing for the GPU): the oracle and
# the .qora-tts reader (csrc/model_file.cpp) with AddressSanitizer and
# UndefinedBehaviorSanitizer, every report fatal.
#   make -f tests/sanitize.mk
# builds tests/_build/liboracle_asan.so and tests/_build/fuzz_model_file;
# tests/test_sanitizers.py runs the reader's fuzz pass and the oracle's CPU
# tests with them.
SAN  = -fsanitize=address,undefined -fno-sanitize-recover=all -fno-omit-frame-pointer -g
ROOT := $(abspath $(dir $(lastword $(MAKEFILE_LIST)))/..)
OUT  = $(ROOT)/tests/_build
ORACLE_SRC = $(ROOT)/oracle/qtts_oracle.c $(ROOT)/oracle/qtts_oracle_decoder.c $(ROOT)/oracle/qtts_oracle_prompt.c
FILE_SRC = $(ROOT)/tests/fuzz_model_file.cpp $(ROOT)/qora-tts-12hz-1.7b_amd/csrc/model_file.cpp

all: $(OUT)/liboracle_asan.so $(OUT)/fuzz_model_file

$(OUT)/liboracle_asan.so: $(ORACLE_SRC) $(ROOT)/oracle/qtts_oracle.h $(ROOT)/include/qtts.h $(ROOT)/include/qtts_decoder.h
	@mkdir -p $(OUT)
	gcc -O1 -std=c11 -fPIC -ffp-contract=off -fno-fast-math $(SAN) -shared -o $@ $(ORACLE_SRC) -lm -lpthread

$(OUT)/fuzz_model_file: $(FILE_SRC) $(ROOT)/include/qtts_file.h $(ROOT)/include/qtts.h $(ROOT)/include/qtts_decoder.h
	@mkdir -p $(OUT)
	g++ -O1 -std=c++17 $(SAN) -o $@ $(FILE_SRC)

clean:
	rm -f $(OUT)/liboracle_asan.so $(OUT)/fuzz_model_file

.PHONY: all clean
