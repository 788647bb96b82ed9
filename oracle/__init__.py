"""CPU oracle for the FP4 delta-CSR sparse layer -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker / the timed CPU baseline.  The
product (sili__new_amd) never imports, links or runs anything here.

    liboracle.so   (_build/)  CPU restatement of the reference (sili_oracle.cpp)
    libsili_ref.so (_ref/)    the reference's own headers compiled in place
                              (only where /root/reference exists at build time)
"""
from .oracle import (  # noqa: F401
    HostLayer, RefLayer, build, dense_to_csr, dense_to_top_k_csr, for_encode_row, for_encode_rows, have_ref, lib,
    ref_for_encode, ref_top_k_csr, reflib, SWITCH_POINT, TileEncodingState, pack_tiles, sparse_pack_tile, tile_live,
    ScatteredReservations, row_content, synap_no_room_message, demote_no_room_message,
    Block4Reservations, block4_row_use, tile_len, tile_len_by_live, uleb_len, Block4PutModel, block4_put_layer,
)
