/* Embeds the gfx950 code object built from csrc/kernels/q4_matvec.hip into
 * libaxh.so; AXH_Q4_MATVEC_CO is the path of that ELF (set by build.py). */
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
    .section .note.GNU-stack,"",@progbits
