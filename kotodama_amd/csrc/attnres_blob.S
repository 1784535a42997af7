/* The eleven gfx950 code-object parts, linked into libattnres_hip.so as bytes
 * and loaded with hipModuleLoadData.  The build passes -I<dir of the .hsaco>. */
    .section .rodata
    .balign 4096
    .global attnres_hsaco_part0
attnres_hsaco_part0:
    .incbin "attnres_gfx950_part0.hsaco"
    .balign 4096
    .global attnres_hsaco_part1
attnres_hsaco_part1:
    .incbin "attnres_gfx950_part1.hsaco"
    .balign 4096
    .global attnres_hsaco_part2
attnres_hsaco_part2:
    .incbin "attnres_gfx950_part2.hsaco"
    .balign 4096
    .global attnres_hsaco_part3
attnres_hsaco_part3:
    .incbin "attnres_gfx950_part3.hsaco"
    .balign 4096
    .global attnres_hsaco_part4
attnres_hsaco_part4:
    .incbin "attnres_gfx950_part4.hsaco"
    .balign 4096
    .global attnres_hsaco_part5
attnres_hsaco_part5:
    .incbin "attnres_gfx950_part5.hsaco"
    .balign 4096
    .global attnres_hsaco_part6
attnres_hsaco_part6:
    .incbin "attnres_gfx950_part6.hsaco"
    .balign 4096
    .global attnres_hsaco_part7
attnres_hsaco_part7:
    .incbin "attnres_gfx950_part7.hsaco"
    .balign 4096
    .global attnres_hsaco_part8
attnres_hsaco_part8:
    .incbin "attnres_gfx950_part8.hsaco"
    .balign 4096
    .global attnres_hsaco_part9
attnres_hsaco_part9:
    .incbin "attnres_gfx950_part9.hsaco"
    .balign 4096
    .global attnres_hsaco_part10
attnres_hsaco_part10:
    .incbin "attnres_gfx950_part10.hsaco"
    .section .note.GNU-stack,"",@progbits
