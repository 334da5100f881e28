/* The chain plan's device code object (chain_plan_kernels.hip, built for
   gfx950 as a plain ELF), embedded read-only in the library. */
    .section .rodata.w4a8_chain_plan_co, "a"
    .p2align 12
    .globl w4a8_chain_plan_co_begin
    .hidden w4a8_chain_plan_co_begin
w4a8_chain_plan_co_begin:
    .incbin W4A8_CHAIN_PLAN_CO
    .globl w4a8_chain_plan_co_end
    .hidden w4a8_chain_plan_co_end
w4a8_chain_plan_co_end:
    .section .note.GNU-stack, "", @progbits
