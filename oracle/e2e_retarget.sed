# Retargets the reference's forward passes (the section between the
# "11 forward passes" and "12 sampling" banners of gemma.c) to the GH_ shims
# of e2e_harness.c: the W8A8 calls and their fp32 twins ('U' model files).  Applied to the source stream while it is piped into the
# compiler; no modified copy of the reference is written anywhere.
/^\/\* 11 forward passes/,/^\/\* 12 sampling/{
s/\bquantize_acts(/GH_quantize_acts(/g
s/\bquantize_act(/GH_quantize_act(/g
s/\bgemv_int8_multi(/GH_gemv_int8_multi(/g
s/\bgemv_int8(/GH_gemv_int8(/g
s/\bgemm_int8(/GH_gemm_int8(/g
s/\bgemv_fpx_multi(/GH_gemv_fpx_multi(/g
s/\bgemv_fpx(/GH_gemv_fpx(/g
s/\bgemm_fpx(/GH_gemm_fpx(/g
}
