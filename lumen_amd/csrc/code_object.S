/* Embeds the gfx950 code object built from sampler_kernels.hip into the
 * host library, so a single .so carries the kernels. */
    .section .rodata
    .balign 4096
    .globl lumen_gfx950_code_object
    .type lumen_gfx950_code_object, @object
lumen_gfx950_code_object:
    .incbin LUMEN_HSACO_PATH
    .globl lumen_gfx950_code_object_end
lumen_gfx950_code_object_end:
    .byte 0
    .section .note.GNU-stack,"",@progbits
