/* Embeds the benchmark's gfx950 code object (bench_kernels.hip) into libglmssd_bench.so. */
    .section .rodata.bn_blob, "a"
    .balign 4096
    .globl bn_blob_start
    .globl bn_blob_end
bn_blob_start:
    .incbin "build/bench_kernels.hsaco"
bn_blob_end:
    .byte 0

.section .note.GNU-stack,"",@progbits
