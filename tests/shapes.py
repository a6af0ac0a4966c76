"""Shape tables for the parity tests, restated as data from the reference's
own test suite (the reference stores no expected values for these shapes;
its tests compare against PyTorch at run time). Expected values here come
from the oracle on the same seeded inputs.
"""

# Testing/test_1.py:228-282 -- (name, N, C, H, W, F, KH, KW, stride, pad)
CONV2D = [
    ("c01", 2, 3, 8, 8, 4, 3, 3, 1, 0),
    ("c02", 2, 3, 8, 8, 4, 5, 5, 1, 0),
    ("c03", 4, 16, 8, 8, 32, 1, 1, 1, 0),
    ("c04", 2, 3, 12, 12, 8, 7, 7, 1, 0),
    ("c05", 2, 3, 8, 8, 4, 3, 3, 1, 1),
    ("c06", 2, 3, 8, 8, 4, 5, 5, 1, 2),
    ("c07", 2, 3, 14, 14, 8, 7, 7, 1, 3),
    ("c08", 2, 3, 8, 8, 4, 3, 3, 2, 0),
    ("c09", 2, 3, 8, 8, 4, 3, 3, 2, 1),
    ("c10", 2, 3, 10, 10, 4, 5, 5, 2, 2),
    ("c11", 2, 4, 12, 12, 8, 3, 3, 3, 1),
    ("c12", 1, 3, 8, 8, 4, 3, 3, 1, 1),
    ("c13", 8, 3, 8, 8, 4, 3, 3, 1, 1),
    ("c14", 32, 3, 8, 8, 4, 3, 3, 1, 1),
    ("c15", 2, 64, 8, 8, 64, 3, 3, 1, 1),
    ("c16", 4, 1, 16, 16, 8, 3, 3, 1, 1),
    ("c17", 4, 8, 8, 8, 1, 3, 3, 1, 1),
    ("c18", 2, 3, 4, 16, 4, 3, 3, 1, 1),
    ("c19", 2, 3, 16, 4, 4, 3, 3, 1, 1),
    ("c20", 2, 4, 8, 8, 8, 1, 3, 1, 0),
    ("c21", 2, 4, 8, 8, 8, 3, 1, 1, 0),
    ("c22", 2, 4, 8, 8, 8, 1, 5, 1, 0),
    ("c23", 2, 3, 32, 32, 8, 3, 3, 1, 1),
    ("c24", 2, 1, 64, 64, 4, 5, 5, 2, 2),
    ("c25", 4, 3, 8, 8, 4, 3, 3, 1, 1),
    ("c26", 4, 3, 8, 8, 4, 3, 3, 2, 1),
    ("c27", 2, 4, 5, 5, 8, 5, 5, 1, 0),    # global conv: kernel == input
    ("c28", 2, 3, 6, 6, 128, 3, 3, 1, 1),
    ("c29", 2, 4, 12, 12, 8, 2, 2, 3, 0),  # stride > kernel: gaps
    # Testing/test_3.py:47-98 -- large conv, 3x3 s2 p1
    ("big_s2", 8, 32, 64, 64, 64, 3, 3, 2, 1),
]

# Shapes that exercise the row-streaming kernels' tiling (not from the
# reference's tests): several and partial 64-channel / 64-filter tiles,
# 3 input-channel chunks, 5x5 taps, rows that are not a multiple of 16
# pixels, two column tiles, a strip split, odd padding.
CONV2D_STREAM = [
    ("s01", 2, 96, 20, 20, 80, 3, 3, 1, 1),    # 2 F tiles (64+16), 2 C tiles for dW, 3 chunks
    ("s02", 3, 16, 24, 24, 24, 5, 5, 1, 2),    # 5x5 forward / dX stream, dW band path
    ("s03", 2, 8, 30, 60, 16, 3, 3, 1, 1),     # 60-pixel rows
    ("s04", 1, 32, 12, 100, 32, 3, 3, 1, 1),   # 2 column tiles (52 + 48)
    ("s05", 2, 24, 64, 32, 40, 3, 3, 1, 1),    # long strips
    ("s06", 2, 16, 16, 16, 16, 3, 3, 1, 0),    # no padding (output 14x14 -> dX stream needs ph=2)
    ("s07", 2, 16, 17, 16, 16, 2, 2, 1, 1),    # even kernel, 18x17 output
    ("s08", 4, 64, 16, 16, 64, 1, 1, 1, 0),    # 1x1: a GEMM over pixels
    ("s09", 2, 16, 8, 64, 16, 1, 3, 1, 1),     # 1x3, one chunk: a single (chunk, row tap) pair, 2 pixel groups
    ("s10", 2, 8, 6, 16, 8, 1, 3, 1, 1),       # 1x3, one chunk, 1 pixel group
    # rows wider than 64 pixels: the stride-1 dW pass in column tiles of 64
    ("s11", 2, 64, 10, 112, 64, 3, 3, 1, 1),   # 2 column tiles (64 + 48)
    ("s12", 1, 16, 9, 200, 24, 3, 3, 1, 1),    # 4 column tiles (64 x 3 + 8), partial filter tile
    ("s13", 2, 16, 6, 144, 16, 1, 3, 1, 1),    # 1x3: no halo rows, 3 column tiles
    ("s14", 1, 72, 5, 68, 8, 3, 3, 1, 1),      # 2 column tiles (64 + 4), 2 channel tiles
    # many small images (images x tiles > two rounds of 256 CUs): the dW
    # strips run across image boundaries
    ("s15", 65, 128, 4, 4, 256, 3, 3, 1, 1),   # 8 tiles, rows of 4 + 2 per image
    ("s16", 130, 64, 5, 8, 256, 3, 3, 1, 1),   # odd image height
    ("s17", 520, 16, 3, 8, 16, 1, 3, 1, 1),    # 1x3: no extra rows per image
    # the last strip's X rows run past the batch's last period: they must
    # read nothing (X ends where its allocation ends)
    ("s20", 64, 256, 14, 16, 256, 3, 3, 1, 1),
    # 64 channels on rows wider than 56: the three-role forward in column tiles
    ("s18", 1, 64, 6, 60, 64, 3, 3, 1, 1),     # 2 tiles of 32 (the second 28 wide)
    ("s19", 2, 64, 5, 200, 40, 3, 3, 1, 1),    # 4 tiles of 52 (the last 44), partial filter tile
    # more than 64 channels on the three-role kernel: one launch per
    # 64-channel slice, each after the first adding to the output (up to 4
    # slice x filter-tile launches, two filter tiles on rows of 56 or more)
    ("m01", 2, 128, 12, 16, 64, 3, 3, 1, 1),   # forward in 2 slices
    ("m02", 1, 192, 6, 60, 64, 3, 3, 1, 1),    # 3 slices, column tiles
    ("m03", 2, 64, 8, 8, 128, 3, 3, 1, 1),     # dX over 128 dY channels: 2 slices
    ("m04", 1, 256, 5, 20, 64, 3, 3, 1, 1),    # 4 slices
    ("m05", 1, 128, 6, 60, 96, 3, 3, 1, 1),    # 2 slices x 2 filter tiles (the second partial)
    ("m06", 1, 128, 4, 64, 128, 3, 3, 1, 1),   # 2 x 2, forward and dX
]

# Edge shapes (not from the reference's tests): 1x1 image and kernel, channel
# counts off the 8/32/64 grid, a tall narrow and a wide image (several column
# tiles), stride 3 with padding 2, a kernel wider than tall, padding larger
# than half the kernel.
CONV2D_EDGE = [
    ("e01", 1, 1, 1, 1, 1, 1, 1, 1, 0),
    ("e02", 2, 300, 5, 5, 7, 3, 3, 1, 1),
    ("e03", 1, 8, 200, 3, 4, 3, 3, 1, 1),
    ("e04", 3, 16, 7, 130, 16, 3, 3, 1, 1),
    ("e05", 2, 5, 17, 19, 3, 3, 3, 3, 2),
    ("e06", 2, 24, 12, 16, 40, 1, 7, 1, 0),
    ("e07", 2, 8, 6, 6, 8, 3, 3, 1, 2),
    ("e08", 1, 65, 9, 9, 129, 3, 3, 2, 1),
    # rows that are not a multiple of 4 floats: the band and row-streaming
    # kernels on copies widened with zero columns (X for the forward, dY for
    # dX, both for dW)
    ("e09", 2, 64, 14, 14, 64, 3, 3, 1, 1),    # 14x14 (a ResNet stage)
    ("e10", 2, 256, 7, 7, 48, 3, 3, 1, 1),     # 7x7, 8 channel chunks, partial filter tile
    ("e11", 2, 128, 28, 28, 64, 3, 3, 2, 1),   # stride 2: dY rows of 14
    ("e12", 3, 16, 11, 13, 24, 3, 3, 1, 1),    # odd height and width
    ("e13", 2, 8, 15, 18, 8, 5, 5, 2, 2),      # 5x5 stride 2: 9-column output
    ("e14", 2, 24, 10, 10, 16, 3, 3, 1, 0),    # no padding: 8-column output from 10
    # 1x1 stride 1 beside 3x3 layers of the same stages (projections)
    ("k01", 3, 256, 14, 14, 64, 1, 1, 1, 0),   # 14-column rows, 256 channels
    ("k02", 2, 64, 7, 8, 256, 1, 1, 1, 0),     # 256 filters
    ("k03", 2, 30, 6, 10, 18, 1, 1, 1, 0),     # channels not a multiple of 8
    # stride 2 with more than 16 taps: the space-to-depth form (4C channels,
    # ceil(R/2) x ceil(S/2) taps, stride 1)
    ("d01", 2, 3, 20, 24, 8, 7, 7, 2, 3),      # a 7x7 stem: all three passes in that form
    ("d02", 2, 5, 17, 21, 16, 5, 5, 2, 2),     # 5x5, 11-column output: forward only
    ("d03", 1, 20, 12, 16, 70, 7, 7, 2, 3),    # 80 channels in that form (3 chunks), 2 filter tiles
]

# Stride-2 shapes for the four-phase and column-parity kernels (not from the
# reference's tests): the dX pass of a stride-2 convolution with 3x3, 4x4 and
# 2x2 kernels, 1-3 channel chunks of dY, two column tiles, partial filter
# tiles, an odd input height.
CONV2D_PHASE2 = [
    ("q01", 2, 24, 16, 48, 96, 3, 3, 2, 1),    # T, U in {1, 2}, 3 chunks
    ("q02", 2, 40, 20, 80, 32, 4, 4, 2, 1),    # 40 phase columns: two column tiles
    ("q03", 3, 16, 12, 16, 64, 2, 2, 2, 0),    # one tap per phase
    # forward 4x4 s2 p1 by column-parity row streaming (32/64 input channels)
    ("q04", 2, 64, 32, 64, 48, 4, 4, 2, 1),    # partial 64-filter tile
    ("q05", 2, 32, 24, 88, 64, 4, 4, 2, 1),    # 44 output columns: two column tiles
    ("q06", 1, 64, 17, 16, 32, 4, 4, 2, 1),    # odd input height
]

# 3x3 s1 p1 64 -> 64 shapes for the fused one-pass backward (not from the
# reference's tests): one-row and odd heights (a strip whose last step has one
# row), one column quad, 24-pixel rows (one 32-pixel K block), 28 and 52
# pixels (two K blocks, an odd quad count), many two-row strips (halo rows
# shared between blocks).
CONV2D_FUSED = [
    ("f01", 1, 64, 1, 56, 64, 3, 3, 1, 1),
    ("f02", 2, 64, 3, 4, 64, 3, 3, 1, 1),
    ("f03", 3, 64, 13, 28, 64, 3, 3, 1, 1),
    ("f04", 2, 64, 20, 52, 64, 3, 3, 1, 1),
    ("f05", 1, 64, 40, 24, 64, 3, 3, 1, 1),
    ("f06", 4, 64, 57, 56, 64, 3, 3, 1, 1),
    # rows wider than 56: column tiles with one quad of dY halo on either side
    ("f07", 1, 64, 7, 200, 64, 3, 3, 1, 1),    # 4 tiles of 52 (the last 44)
    ("f08", 2, 64, 9, 112, 64, 3, 3, 1, 1),    # 2 tiles of 56
]

# Testing/test_1.py:398-470 -- (name, N, Cin, H, W, Cout, KH, KW, stride, pad)
CONVT = [
    ("t01", 2, 4, 4, 4, 8, 3, 3, 1, 0),
    ("t02", 2, 4, 4, 4, 8, 3, 3, 1, 1),
    ("t03", 2, 4, 4, 4, 8, 5, 5, 1, 2),
    ("t04", 4, 16, 8, 8, 8, 1, 1, 1, 0),
    ("t05", 2, 4, 4, 4, 8, 3, 3, 2, 0),
    ("t06", 2, 4, 4, 4, 8, 4, 4, 2, 1),
    ("t07", 2, 8, 4, 4, 4, 3, 3, 2, 1),
    ("t08", 2, 4, 4, 4, 4, 2, 2, 2, 0),
    ("t09", 2, 4, 3, 3, 4, 3, 3, 3, 0),
    ("t10", 1, 4, 4, 4, 8, 3, 3, 2, 1),
    ("t11", 16, 4, 4, 4, 8, 3, 3, 2, 1),
    ("t12", 2, 64, 4, 4, 32, 3, 3, 2, 1),
    ("t13", 2, 1, 8, 8, 8, 3, 3, 2, 1),
    ("t14", 2, 8, 4, 4, 1, 3, 3, 2, 1),
    ("t15", 2, 4, 2, 8, 8, 3, 3, 2, 1),
    ("t16", 2, 4, 8, 2, 8, 3, 3, 2, 1),
    ("t17", 2, 4, 4, 4, 8, 1, 3, 1, 0),
    ("t18", 2, 4, 4, 4, 8, 3, 1, 1, 0),
    ("t19", 2, 4, 4, 4, 8, 3, 3, 2, 1),
    # Testing/test_3.py:100-136 -- large convT, 4x4 s2 p1
    ("big_t", 8, 64, 32, 32, 32, 4, 4, 2, 1),
]

# Transposed shapes for the four-phase kernel (not from the reference's
# tests): one and three input-channel chunks, 36 phase columns (two column
# tiles), 40 output channels (a partial 32-filter tile), a 2x2 kernel; and
# input rows of 7 and 9 columns (the widened-copy path).
CONVT_PHASE2 = [
    ("u01", 2, 32, 6, 20, 40, 4, 4, 2, 1),
    ("u02", 2, 96, 10, 36, 24, 4, 4, 2, 1),
    ("u03", 3, 64, 8, 8, 16, 2, 2, 2, 0),
    ("u04", 1, 128, 28, 28, 64, 4, 4, 2, 1),   # one image of config 5
    ("u05", 2, 96, 14, 20, 32, 4, 4, 2, 1),    # dX by column-parity streaming, one chunk
    ("u06", 2, 64, 7, 7, 32, 4, 4, 2, 1),      # 7-column input rows (widened copy)
    ("u07", 2, 32, 5, 9, 16, 3, 3, 2, 1),      # 3x3 s2, odd widths both ways
]

# (M, K, N, Nbatch): Testing/test_2.py:372-375, Testing/test_14.py:148-183,
# Testing/diagnose_sizes.py:17-32, Testing/test_2.py:660-663 (dense layers),
# Testing/diagnose_gpu_ops.py:77-107 (manual backward at M=4, K=3, N=2).
MATMUL = [
    (8, 8, 8, 1), (16, 4, 8, 1), (4, 32, 16, 1), (32, 64, 10, 1),
    (8, 16, 6, 1), (33, 65, 17, 1), (4, 10, 5, 1), (8, 128, 5, 1),
    (1, 1, 1, 1), (2, 3, 4, 1), (16, 32, 16, 1), (64, 256, 128, 1),
    (4, 3, 2, 1), (128, 128, 128, 1), (100, 200, 300, 1),
    (7, 13, 5, 3), (16, 16, 16, 4), (33, 17, 65, 2),
    # MLP 784->512->256->10 at batch 256: fwd shapes
    (256, 784, 512, 1), (256, 512, 256, 1), (256, 256, 10, 1),
    # Dense 64x784x128
    (64, 784, 128, 1),
    # not from the reference's tests: 64x64 tiles over a contraction of at
    # least 512 (two wave groups, each over half of it), with a K tail
    (512, 1057, 1000, 1), (1000, 1100, 1000, 1), (768, 600, 768, 1), (896, 777, 640, 1),
    # few tiles: two wave groups in place of a three- or four-way split-K, the
    # last group's part a K tail
    (256, 400, 256, 1), (256, 500, 256, 1),
    # 32x32 tiles (one wave per K group): 8, 4 and 2 groups, a scalar-load B,
    # a backward pair on 32x32 tiles and one that retries on 64x64 ones
    (64, 1200, 64, 1), (96, 1536, 96, 1), (160, 600, 72, 1), (50, 300, 30, 2),
]

# Testing/test_1.py:309-340 -- (name, N, C, H, W, KH, KW, stride, pad), MaxPool2D
MAXPOOL = [
    ("p01", 2, 4, 8, 8, 2, 2, 2, 0),
    ("p02", 2, 4, 9, 9, 3, 3, 3, 0),
    ("p03", 2, 4, 16, 16, 4, 4, 4, 0),
    ("p04", 2, 4, 8, 8, 2, 2, 1, 0),
    ("p05", 2, 4, 8, 8, 3, 3, 2, 0),
    ("p06", 2, 4, 8, 8, 3, 3, 1, 0),
    ("p07", 2, 4, 8, 8, 2, 2, 2, 1),
    ("p08", 2, 4, 8, 8, 3, 3, 2, 1),
    ("p09", 1, 8, 8, 8, 2, 2, 2, 0),
    ("p10", 16, 8, 8, 8, 2, 2, 2, 0),
    ("p11", 2, 64, 8, 8, 2, 2, 2, 0),
    ("p12", 2, 1, 8, 8, 2, 2, 2, 0),
    ("p13", 2, 4, 4, 16, 2, 2, 2, 0),
    ("p14", 2, 4, 16, 4, 2, 2, 2, 0),
    ("p15", 2, 4, 32, 32, 2, 2, 2, 0),
    ("p16", 2, 4, 64, 64, 4, 4, 4, 0),
    ("p17", 4, 8, 4, 4, 4, 4, 4, 0),
    # not from the reference's tests: stride > kernel (gaps), padding >= the
    # window (windows wholly in the padding), an odd extent that the stride
    # does not divide
    ("q01", 2, 3, 11, 11, 2, 2, 3, 0),
    ("q02", 1, 2, 5, 7, 2, 2, 1, 2),
    ("q03", 2, 3, 13, 10, 3, 3, 2, 1),
    ("q04", 2, 3, 9, 10, 2, 2, 2, 0),    # 2x2 s2, odd H: a tail row under the last windows
    ("q05", 2, 3, 8, 9, 2, 2, 2, 0),     # 2x2 s2, odd W: a tail column
    ("q06", 2, 3, 10, 11, 4, 4, 1, 1),   # 4 windows cover an element per axis: loop kernels
]
