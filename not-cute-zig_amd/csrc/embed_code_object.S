/* Embeds the gfx950 code object built from flash_fwd.hip into the host library, the counterpart
   of the reference's @embedFile("cuda-module") (build.zig:94-101, src/main.zig:32). */
    .section .rodata.nc_code_object,"a",@progbits
    .p2align 12
    .globl nc_embedded_code_object
    .type nc_embedded_code_object, @object
nc_embedded_code_object:
    .incbin "flash_fwd_gfx950.hsaco"
    .globl nc_embedded_code_object_end
nc_embedded_code_object_end:
    .byte 0
    .section .note.GNU-stack,"",@progbits
