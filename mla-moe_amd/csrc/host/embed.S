/* embed.S -- the gfx950 code objects built from csrc/kernels/*.hip, linked
 * into libmlamoe.so as read-only data and loaded with hipModuleLoadData.
 * The assembler finds the .hsaco files through -I<build dir>. */
    .section .rodata.mm_code_objects, "a", @progbits

    .balign 4096
    .globl mm_co_moe_bf16
    .hidden mm_co_moe_bf16
    .type mm_co_moe_bf16, @object
mm_co_moe_bf16:
    .incbin "moe_bf16.hsaco"

    .balign 4096
    .globl mm_co_util
    .hidden mm_co_util
    .type mm_co_util, @object
mm_co_util:
    .incbin "util.hsaco"

    .balign 4096
    .globl mm_co_moe_i8
    .hidden mm_co_moe_i8
    .type mm_co_moe_i8, @object
mm_co_moe_i8:
    .incbin "moe_i8.hsaco"

    .balign 4096
    .globl mm_co_mla
    .hidden mm_co_mla
    .type mm_co_mla, @object
mm_co_mla:
    .incbin "mla.hsaco"

    .balign 4096
    .globl mm_co_gemm_bf16
    .hidden mm_co_gemm_bf16
    .type mm_co_gemm_bf16, @object
mm_co_gemm_bf16:
    .incbin "gemm_bf16.hsaco"

    .balign 4096
    .globl mm_co_gemm_i8
    .hidden mm_co_gemm_i8
    .type mm_co_gemm_i8, @object
mm_co_gemm_i8:
    .incbin "gemm_i8.hsaco"

    .balign 4096
    .globl mm_co_lm_head
    .hidden mm_co_lm_head
    .type mm_co_lm_head, @object
mm_co_lm_head:
    .incbin "lm_head.hsaco"

    .balign 4096
    .globl mm_co_gemv
    .hidden mm_co_gemv
    .type mm_co_gemv, @object
mm_co_gemv:
    .incbin "gemv.hsaco"

    .section .note.GNU-stack, "", @progbits
