/* Embeds the gfx950 code objects built from attn_kernels.hip (one per kernel
 * part, TMAC_PART = 0..3) into libtmac_attn.so; tmac_init loads each with
 * hipModuleLoadData.  tmac_attn_code_objects[i] / _sizes[i] describe part i. */
.macro TMAC_BLOB n
    .section .rodata.tmac_attn_code_object_\n,"a",@progbits
    .p2align 12
.Ltmac_blob_\n:
    .incbin "attn_kernels_\n\().hsaco"
.Ltmac_blob_end_\n:
.endm
    TMAC_BLOB 0
    TMAC_BLOB 1
    TMAC_BLOB 2
    TMAC_BLOB 3

    .section .data.rel.ro.tmac_attn_code_objects,"aw",@progbits
    .globl tmac_attn_code_objects
    .type tmac_attn_code_objects, @object
    .p2align 3
tmac_attn_code_objects:
    .quad .Ltmac_blob_0, .Ltmac_blob_1, .Ltmac_blob_2, .Ltmac_blob_3
    .size tmac_attn_code_objects, 32

    .section .rodata.tmac_attn_code_object_sizes,"a",@progbits
    .globl tmac_attn_code_object_sizes
    .type tmac_attn_code_object_sizes, @object
    .p2align 3
tmac_attn_code_object_sizes:
    .quad .Ltmac_blob_end_0 - .Ltmac_blob_0, .Ltmac_blob_end_1 - .Ltmac_blob_1
    .quad .Ltmac_blob_end_2 - .Ltmac_blob_2, .Ltmac_blob_end_3 - .Ltmac_blob_3
    .size tmac_attn_code_object_sizes, 32

    .section .note.GNU-stack,"",@progbits
