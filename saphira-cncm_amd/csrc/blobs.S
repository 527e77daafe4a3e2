/* blobs.S -- embeds the gfx950 code objects built from csrc/*.hip into
 * libncmhip.so; runtime.c hands them to hipModuleLoadData. */
    .section .rodata
    .balign 4096
    .globl ncm_co_gemm
ncm_co_gemm:
    .incbin "gemm.co"
    .balign 4096
    .globl ncm_co_vq
ncm_co_vq:
    .incbin "vq.co"
    .balign 4096
    .globl ncm_co_ops
ncm_co_ops:
    .incbin "ops.co"
    .balign 4096
    .globl ncm_co_train
ncm_co_train:
    .incbin "train.co"
    .balign 4096
    .globl ncm_co_sample
ncm_co_sample:
    .incbin "sample.co"
    .balign 4096
    .globl ncm_co_ncp
ncm_co_ncp:
    .incbin "ncp.co"
    .section .note.GNU-stack,"",@progbits
