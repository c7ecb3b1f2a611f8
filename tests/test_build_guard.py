"""The build's assembly checks (CPU): the store-data hazard scan flags a
16-byte store whose data registers a VALU instruction rewrites within two
wait states, and passes the same code once two instructions separate them."""
from glt_amd.build import store_data_hazards


def test_store_data_hazard_scan():
    # the pair the compiler emitted for the masked-CE gradient stores: the
    # store's first data register rewritten by the next instruction (the
    # scheduling barrier between them emits no code)
    bad = ("\tbuffer_store_dwordx4 v[50:53], v1, s[4:7], s38 offen\n"
           "\t; sched_barrier mask(0x00000000)\n"
           "\tv_lshlrev_b32_e32 v50, 16, v46\n")
    assert len(store_data_hazards(bad)) == 1
    # two scalar instructions in between: the two wait states are there
    ok = ("\tbuffer_store_dwordx4 v[66:69], v76, s[4:7], 0 offen\n"
          "\ts_cmp_eq_u32 s20, 2\n"
          "\ts_cselect_b64 s[10:11], -1, 0\n"
          "\tv_mul_f32_e32 v67, v71, v78\n")
    assert store_data_hazards(ok) == []
    # one wait state is not enough; a write of other registers is no hazard
    short = "\tglobal_store_dwordx4 v[2:3], v[8:11], off\n\ts_nop 0\n\tv_mov_b32_e32 v9, 0\n"
    assert len(store_data_hazards(short)) == 1
    other = "\tbuffer_store_dwordx4 v[8:11], v1, s[4:7], s3 offen\n\tv_mov_b32_e32 v12, 0\n"
    assert store_data_hazards(other) == []
    # an 8-byte store has no such hazard
    small = "\tbuffer_store_dwordx2 v[8:9], v1, s[4:7], s3 offen\n\tv_mov_b32_e32 v8, 0\n"
    assert store_data_hazards(small) == []
