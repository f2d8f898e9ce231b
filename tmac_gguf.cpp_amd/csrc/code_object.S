/* Embeds the gfx950 code object built from attn_kernels.hip into
 * libtmac_attn.so; tmac_init passes it to hipModuleLoadData. */
    .section .rodata.tmac_attn_code_object,"a",@progbits
    .globl tmac_attn_code_object
    .type tmac_attn_code_object, @object
    .p2align 12
tmac_attn_code_object:
    .incbin "attn_kernels.hsaco"
.Ltmac_attn_code_object_end:
    .size tmac_attn_code_object, .Ltmac_attn_code_object_end - tmac_attn_code_object

    .globl tmac_attn_code_object_size
    .type tmac_attn_code_object_size, @object
    .p2align 3
tmac_attn_code_object_size:
    .quad .Ltmac_attn_code_object_end - tmac_attn_code_object
    .size tmac_attn_code_object_size, 8

    .section .note.GNU-stack,"",@progbits
