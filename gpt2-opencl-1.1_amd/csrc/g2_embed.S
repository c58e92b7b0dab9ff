/* g2_embed.S -- links the gfx950 code object (built from g2_kernels.hip)
 * into libg2hip.so as read-only data for hipModuleLoadData. */
    .section .rodata
    .p2align 12
    .globl g2_hsaco_begin
    .type g2_hsaco_begin, @object
g2_hsaco_begin:
    .incbin G2_HSACO_PATH
    .globl g2_hsaco_end
    .type g2_hsaco_end, @object
g2_hsaco_end:
    .byte 0
    .section .note.GNU-stack,"",@progbits
