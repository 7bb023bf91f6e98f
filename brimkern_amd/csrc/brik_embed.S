/* Embeds the gfx950 code object (built by hipcc --genco) into libbrik.so. */
    .section .rodata.brik_hsaco, "a"
    .balign 4096
    .globl brik_hsaco_begin
    .type brik_hsaco_begin, @object
brik_hsaco_begin:
    .incbin BRIK_HSACO_PATH
    .globl brik_hsaco_end
brik_hsaco_end:
    .byte 0
    .section .note.GNU-stack, "", @progbits
