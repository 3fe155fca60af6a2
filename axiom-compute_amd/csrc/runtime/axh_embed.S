/* Embeds the gfx950 code objects built from csrc/kernels/q4_matvec.hip and
 * csrc/kernels/q4_matmul.hip into libaxh.so; AXH_Q4_MATVEC_CO and
 * AXH_Q4_MATMUL_CO are the paths of those ELFs (set by build.py). */
    .section .rodata
    .balign 4096
    .global axh_q4_matvec_co_begin
    .type axh_q4_matvec_co_begin, @object
axh_q4_matvec_co_begin:
    .incbin AXH_Q4_MATVEC_CO
    .global axh_q4_matvec_co_end
    .type axh_q4_matvec_co_end, @object
axh_q4_matvec_co_end:
    .byte 0
    .balign 4096
    .global axh_q4_matmul_co_begin
    .type axh_q4_matmul_co_begin, @object
axh_q4_matmul_co_begin:
    .incbin AXH_Q4_MATMUL_CO
    .global axh_q4_matmul_co_end
    .type axh_q4_matmul_co_end, @object
axh_q4_matmul_co_end:
    .byte 0
    .section .note.GNU-stack,"",@progbits
