! fgpt_run.f90 -- ids-in / ids-out harness over the drop-in model API.
!
! Reproduces the call semantics of the reference's inference apps with the
! gfx950 engine underneath:
!   greedy   the decode loop of src/app/chat_text.f90:225-278,423-462: RoPE
!            tables built on the host in fp32, the prompt (minus its last id)
!            through gpt_step_multi chunks of pchunk, then one gpt_step per
!            generated id with a host argmax (src/lib/sample.f90:271-277,
!            first maximum; no byte mask). With loop=device the generated
!            ids come from the engine's device-side greedy loop instead.
!   eval     the per-position NLL of src/app/eval_bpb.f90:117-126,156-181:
!            B rows of T+1 ids, gpt_forward on the first T, nats per
!            position = logsumexp - logit[target].
!   bpb      eval_bpb + bpb_agg on the device (src/app/eval_bpb.f90:97-181,
!            src/app/bpb_agg.f90): an int32 (N, T+1) rows .npy, batch rows
!            per forward, nats weighted by a token byte-length table (one
!            int per line, token id order); prints bpb_agg's summary line,
!            and eval_bpb's per-position NLL lines to NLL_OUT when given.
!   spec     greedy speculative decoding as chat_text --spec runs it
!            (src/app/chat_text.f90:293-422: prompt-lookup drafts, one
!            verification pass per round, the sliding-window controller),
!            checked against a plain greedy run on a second cache as
!            src/app/spec_bench.f90 does; prints its summary lines.
!   sample   chat_text's plain loop with sample_next (src/app/chat_text.f90:
!            423-462, src/lib/sample.f90:153-233): loop=host steps through the
!            drop-in gpt_step and sample_next, loop=device is one
!            fg_decode_sample call; the history is the ids generated so far.
!   (The drop-in checks -- cached steps == forward, spec_bench's
!   truncated-drafter run, eval_bpb's --attn blas statistics -- are the
!   program tests/fortran/dropin_checks.f90.)
!
! Usage:
!   fgpt_run greedy WDIR L D H KH HD V IDS_FILE NGEN OUT_FILE [PCHUNK] [host|device]
!   fgpt_run eval   WDIR L D H KH HD V ROWS_FILE B T OUT_FILE [f16]
!   fgpt_run bpb    WDIR L D H KH HD V ROWS_NPY TOKEN_BYTES [BATCH] [NLL_OUT]
!   fgpt_run spec   WDIR L D H KH HD V IDS_FILE NGEN OUT_FILE [K] [MATCH] [PROBE] [MIN_ACC]
!   fgpt_run sample WDIR L D H KH HD V IDS_FILE NGEN OUT_FILE TEMP TOPP SEED
!                   [PRES FREQ REP PWIN PLEN NBLOCK BYTE(0|1) [host|device]]
! Ids files are whitespace-separated 0-based integers. Timing goes to stderr.
program fgpt_run
  use, intrinsic :: iso_c_binding
  use, intrinsic :: iso_fortran_env, only: error_unit, int64
  use fgpt_c
  use fgpt_drop_in_mod
  use fgpt_util
  implicit none

  character(len=512) :: mode
  integer :: nargs

  nargs = command_argument_count()
  if (nargs < 1) call usage()
  call get_command_argument(1, mode)
  select case (trim(mode))
  case ('greedy')
    call run_greedy()
  case ('eval')
    call run_eval()
  case ('bpb')
    call run_bpb()
  case ('spec')
    call run_spec()
  case ('sample')
    call run_sample()
  case default
    call usage()
  end select

contains

  subroutine usage()
    write (error_unit, '(A)') 'usage: fgpt_run greedy WDIR L D H KH HD V IDS NGEN OUT [PCHUNK] [host|device]'
    write (error_unit, '(A)') '       fgpt_run eval WDIR L D H KH HD V ROWS B T OUT'
    write (error_unit, '(A)') '       fgpt_run bpb WDIR L D H KH HD V ROWS_NPY TOKEN_BYTES [BATCH] [NLL_OUT]'
    write (error_unit, '(A)') '       fgpt_run spec WDIR L D H KH HD V IDS NGEN OUT [K] [MATCH] [PROBE] [MIN_ACC]'
    write (error_unit, '(A)') '       fgpt_run sample WDIR L D H KH HD V IDS NGEN OUT TEMP TOPP SEED ' // &
        '[PRES FREQ REP PWIN PLEN NBLOCK BYTE [host|device]]'
    stop 2
  end subroutine usage

  subroutine run_greedy()
    character(len=512) :: wdir, ids_file, out_file, loop
    integer :: L, D, H, KH, HD, V, ngen, pchunk, nprompt, ntot, npre, srow, tb, step, tc, i, u, best
    integer(c_int) :: clen
    real(c_float), allocatable :: wte(:), lm(:), c_q(:), c_k(:), c_v(:), c_pr(:), c_fc(:), c_pr2(:)
    real(c_float), allocatable :: cos_b(:), sin_b(:), out1(:), outc(:), ck(:), cv(:)
    integer(c_int), allocatable :: prompt(:), idx(:), gen(:)
    type(c_ptr) :: model, kv
    integer(c_int32_t) :: rc
    real(8) :: t0, t1, t2

    if (command_argument_count() < 11) call usage()
    wdir = sarg(2); L = iarg(3); D = iarg(4); H = iarg(5); KH = iarg(6); HD = iarg(7); V = iarg(8)
    ids_file = sarg(9); ngen = iarg(10); out_file = sarg(11)
    pchunk = 64
    if (command_argument_count() >= 12) pchunk = iarg(12)
    loop = 'host'
    if (command_argument_count() >= 13) loop = sarg(13)

    call load_gpt_weights(trim(wdir), L, D, H, KH, HD, V, wte, lm, c_q, c_k, c_v, c_pr, c_fc, c_pr2)
    call read_ids(trim(ids_file), prompt, nprompt)
    if (nprompt < 1) then
      write (error_unit, '(A)') 'empty prompt'
      stop 1
    end if
    ntot = nprompt + ngen
    allocate (idx(ntot), out1(V), ck(1), cv(1))
    idx(1:nprompt) = prompt(1:nprompt)
    call rope_tables(ntot, HD, cos_b, sin_b)
    clen = 0

    t0 = now()
    npre = nprompt - 1
    if (npre >= 1) then
      allocate (outc(max(1, min(pchunk, npre))*V))
      srow = 1
      do while (srow <= npre)
        tb = min(pchunk, npre - srow + 1)
        call gpt_step_multi(idx(srow:srow+tb-1), cos_b((srow-1)*(HD/2)+1:), &
            sin_b((srow-1)*(HD/2)+1:), wte, c_q, c_k, c_v, c_pr, c_fc, c_pr2, lm, &
            ck, cv, clen, ntot, outc, 1, V, D, H, KH, HD, L, tb, 1.0e-5_c_float)
        srow = srow + tb
      end do
    end if
    t1 = now()
    if (trim(loop) == 'device') then
      ! one host call: the engine feeds each argmax back on the device
      if (npre < 1) then
        ! bind the model and cache through a zero-length-free first step
        call gpt_step(idx(1:1), cos_b, sin_b, wte, c_q, c_k, c_v, c_pr, c_fc, c_pr2, lm, &
            ck, cv, clen, ntot, out1, 1, V, D, H, KH, HD, L, 1.0e-5_c_float)
        best = 1
        do i = 2, V
          if (out1(i) > out1(best)) best = i
        end do
        idx(nprompt+1) = best - 1
        call fgpt_handles(model, kv)
        call set_rope_rows(model, clen, ngen - 1, HD, cos_b, sin_b)
        allocate (gen(max(ngen-1, 1)))
        if (ngen > 1) then
          rc = fg_decode_greedy(model, kv, idx(nprompt+1:nprompt+1), ngen-1, gen, c_null_ptr)
          if (rc /= FG_OK) then
            write (error_unit, '(2A)') 'fg_decode_greedy: ', fg_error_message()
            stop 1
          end if
          idx(nprompt+2:ntot) = gen(1:ngen-1)
        end if
      else
        call fgpt_handles(model, kv)
        call set_rope_rows(model, clen, ngen, HD, cos_b, sin_b)
        allocate (gen(ngen))
        rc = fg_decode_greedy(model, kv, idx(nprompt:nprompt), ngen, gen, c_null_ptr)
        if (rc /= FG_OK) then
          write (error_unit, '(2A)') 'fg_decode_greedy: ', fg_error_message()
          stop 1
        end if
        idx(nprompt+1:ntot) = gen(1:ngen)
      end if
    else
      do step = nprompt, ntot - 1
        tc = step
        call gpt_step(idx(tc:tc), cos_b((tc-1)*(HD/2)+1:), sin_b((tc-1)*(HD/2)+1:), &
            wte, c_q, c_k, c_v, c_pr, c_fc, c_pr2, lm, ck, cv, clen, ntot, out1, &
            1, V, D, H, KH, HD, L, 1.0e-5_c_float)
        if (out1(1) /= out1(1)) then
          print '(A)', "NaN logit - abort"
          stop 1
        end if
        best = 1
        do i = 2, V
          if (out1(i) > out1(best)) best = i
        end do
        idx(tc+1) = best - 1
      end do
    end if
    t2 = now()
    open (newunit=u, file=trim(out_file), status='replace', action='write')
    do i = nprompt + 1, ntot
      write (u, '(I0)') idx(i)
    end do
    close (u)
    write (error_unit, '(A,F10.3,A,F10.3,A,F12.1,2A)') 'stats: prefill_ms=', 1000*(t1-t0), &
        ' decode_ms=', 1000*(t2-t1), ' tok_s=', real(ngen, 8)/max(t2-t1, 1d-9), ' loop=', trim(loop)
    call fgpt_release()
  end subroutine run_greedy

  subroutine run_eval()
    character(len=512) :: wdir, rows_file, out_file
    integer :: L, D, H, KH, HD, V, B, T, n, r, tcc, j, u, tgt, base
    real(c_float), allocatable :: wte(:), lm(:), c_q(:), c_k(:), c_v(:), c_pr(:), c_fc(:), c_pr2(:)
    real(c_float), allocatable :: cos_b(:), sin_b(:), outp(:), nll(:,:)
    integer(c_int), allocatable :: rows(:), idx(:)
    real(c_float) :: m, s
    real(8) :: t0, t1, tot

    if (command_argument_count() < 12) call usage()
    wdir = sarg(2); L = iarg(3); D = iarg(4); H = iarg(5); KH = iarg(6); HD = iarg(7); V = iarg(8)
    rows_file = sarg(9); B = iarg(10); T = iarg(11); out_file = sarg(12)
    ! f16: the single-term fp16 forward (fgpt_forward_f16), as eval_bpb may ask for it
    if (command_argument_count() >= 13) call fgpt_forward_f16(trim(sarg(13)) == 'f16')
    call load_gpt_weights(trim(wdir), L, D, H, KH, HD, V, wte, lm, c_q, c_k, c_v, c_pr, c_fc, c_pr2)
    call read_ids(trim(rows_file), rows, n)
    if (n /= B*(T+1)) then
      write (error_unit, '(A,I0,A,I0)') 'rows file holds ', n, ' ids, need ', B*(T+1)
      stop 1
    end if
    allocate (idx(B*T), outp(B*T*V), nll(B, T))
    do r = 1, B
      idx((r-1)*T+1:r*T) = rows((r-1)*(T+1)+1:(r-1)*(T+1)+T)
    end do
    call rope_tables(T, HD, cos_b, sin_b)
    t0 = now()
    call gpt_forward(idx, cos_b, sin_b, wte, c_q, c_k, c_v, c_pr, c_fc, c_pr2, lm, outp, &
        B, T, V, D, H, KH, HD, L, 1.0e-5_c_float)
    t1 = now()
    do r = 1, B
      base = (r-1)*T*V
      do tcc = 1, T
        tgt = rows((r-1)*(T+1) + tcc + 1) + 1
        m = outp(base+(tcc-1)*V+1)
        do j = 2, V
          if (outp(base+(tcc-1)*V+j) > m) m = outp(base+(tcc-1)*V+j)
        end do
        s = 0.0_c_float
        do j = 1, V
          s = s + exp(outp(base+(tcc-1)*V+j) - m)
        end do
        nll(r, tcc) = (m + log(s)) - outp(base+(tcc-1)*V+tgt)
      end do
    end do
    open (newunit=u, file=trim(out_file), status='replace', action='write')
    do r = 1, B
      tot = 0
      do tcc = 1, T
        tot = tot + nll(r, tcc)
      end do
      write (u, '(ES24.16)') tot
    end do
    close (u)
    write (error_unit, '(A,F10.3,A,F14.1)') 'stats: forward_ms=', 1000*(t1-t0), &
        ' tok_s=', real(B*T, 8)/max(t1-t0, 1d-9)
    call fgpt_release()
    call fgpt_forward_f16(.false.)
  end subroutine run_eval

  subroutine run_bpb()
    character(len=512) :: wdir, rows_file, tb_file, nll_file
    integer :: L, D, H, KH, HD, V, batch, u, ios, ntb, r, tc
    integer(c_int32_t) :: rc, nrows, width, T
    integer(c_int32_t), allocatable, target :: rows(:)
    integer(c_int32_t), allocatable :: tb(:), tmp(:)
    real(c_float), allocatable :: cos_b(:), sin_b(:), nll(:)
    real(c_double), allocatable :: rn(:)
    integer(c_int64_t), allocatable :: rb(:)
    real(c_double) :: tn
    integer(c_int64_t) :: tbt
    type(c_ptr) :: model
    type(fg_dims) :: fd
    real(8) :: t0, t1

    if (command_argument_count() < 10) call usage()
    wdir = sarg(2); L = iarg(3); D = iarg(4); H = iarg(5); KH = iarg(6); HD = iarg(7); V = iarg(8)
    rows_file = sarg(9); tb_file = sarg(10)
    batch = 8
    if (command_argument_count() >= 11) batch = iarg(11)
    nll_file = ''
    if (command_argument_count() >= 12) nll_file = sarg(12)

    rc = fg_rows_npy(trim(rows_file)//c_null_char, nrows, width, c_null_ptr)
    if (rc /= FG_OK) call stop_rc('rows', rc)
    T = width - 1
    allocate (rows(int(nrows)*int(width)))
    rc = fg_rows_npy(trim(rows_file)//c_null_char, nrows, width, c_loc(rows))
    if (rc /= FG_OK) call stop_rc('rows', rc)

    ! token byte lengths: one integer per line, id order (bpb_agg.f90:63-84)
    allocate (tmp(1048576))
    ntb = 0
    open (newunit=u, file=trim(tb_file), status='old', action='read', iostat=ios)
    if (ios /= 0) then
      write (error_unit, '(2A)') 'cannot open ', trim(tb_file)
      stop 2
    end if
    do
      if (ntb >= size(tmp)) exit
      read (u, *, iostat=ios) tmp(ntb + 1)
      if (ios /= 0) exit
      ntb = ntb + 1
    end do
    close (u)
    if (ntb == 0) then
      write (error_unit, '(A)') 'empty token_bytes'
      stop 2
    end if
    tb = tmp(1:ntb)

    fd = fg_dims(L, D, H, KH, HD, V, 1.0e-5_c_float)
    rc = fg_model_load(fd, trim(wdir)//c_null_char, model)
    if (rc /= FG_OK) call stop_rc('fg_model_load', rc)
    call rope_tables(int(T), HD, cos_b, sin_b)
    call set_rope_rows(model, 0, int(T), HD, cos_b, sin_b)
    allocate (nll(int(nrows)*int(T)), rn(nrows), rb(nrows))
    t0 = now()
    rc = fg_eval_bpb(model, rows, nrows, T, int(batch, c_int32_t), tb, int(ntb, c_int32_t), nll, &
        rn, rb, tn, tbt)
    t1 = now()
    if (rc /= FG_OK) call stop_rc('fg_eval_bpb', rc)
    if (len_trim(nll_file) > 0) then
      open (newunit=u, file=trim(nll_file), status='replace', action='write')
      do r = 1, nrows
        do tc = 1, T
          if (tc > 1) write (u, '(A)', advance='no') ' '
          write (u, '(ES14.7)', advance='no') nll((r - 1)*T + tc)
        end do
        write (u, *)
      end do
      close (u)
    end if
    do r = 1, nrows
      if (rb(r) > 0) write (*, '(A,I0,A,F0.4)') 'row ', r - 1, ': bpb=', rn(r)/(log(2.0d0)*rb(r))
    end do
    if (tbt == 0) then
      write (error_unit, '(A)') 'no counted bytes'
      stop 1
    end if
    write (*, '(A,I0,A,I0,A,F0.2,A,F0.5)') 'rows=', nrows, ' bytes=', tbt, ' nll_sum=', tn, &
        ' bpb=', tn / real(tbt, 8) / log(2.0d0)
    write (error_unit, '(A,F10.3,A,F14.1)') 'stats: eval_ms=', 1000*(t1 - t0), &
        ' tok_s=', real(nrows, 8)*T/max(t1 - t0, 1d-9)
    rc = fg_model_destroy(model)
  end subroutine run_bpb

  subroutine run_spec()
    character(len=512) :: wdir, ids_file, out_file
    integer :: L, D, H, KH, HD, V, ngen, nprompt, ntot, srow, tb, u, i
    integer(c_int32_t) :: rc
    integer(c_int), allocatable :: prompt(:)
    integer(c_int32_t), allocatable :: ids(:), plain(:)
    real(c_float), allocatable :: cos_b(:), sin_b(:), lg(:)
    type(c_ptr) :: model, kv, kv2
    type(fg_dims) :: fd
    type(fg_spec_cfg) :: cfg
    type(fg_spec_stats) :: st
    real(8) :: t0, t1, t2

    if (command_argument_count() < 11) call usage()
    wdir = sarg(2); L = iarg(3); D = iarg(4); H = iarg(5); KH = iarg(6); HD = iarg(7); V = iarg(8)
    ids_file = sarg(9); ngen = iarg(10); out_file = sarg(11)
    ! chat_text's defaults for --match / --spec-probe / --spec-min-acc
    cfg = fg_spec_cfg(8, 2, 8, 0.5_c_float)
    if (command_argument_count() >= 12) cfg%k = iarg(12)
    if (command_argument_count() >= 13) cfg%match = iarg(13)
    if (command_argument_count() >= 14) cfg%probe = iarg(14)
    if (command_argument_count() >= 15) cfg%min_acc = real(rarg(15), c_float)
    call read_ids(trim(ids_file), prompt, nprompt)
    if (nprompt < 1) then
      write (error_unit, '(A)') 'empty prompt'
      stop 1
    end if
    ntot = nprompt + ngen
    fd = fg_dims(L, D, H, KH, HD, V, 1.0e-5_c_float)
    rc = fg_model_load(fd, trim(wdir)//c_null_char, model)
    if (rc /= FG_OK) call stop_rc('fg_model_load', rc)
    call rope_tables(ntot, HD, cos_b, sin_b)
    call set_rope_rows(model, 0, ntot, HD, cos_b, sin_b)
    allocate (ids(ntot), plain(max(ngen, 1)), lg(64*V))
    ids(1:nprompt) = prompt(1:nprompt)

    ! plain greedy on its own cache (spec_bench's run_plain): the per-kernel
    ! steps, whose arithmetic the verification pass repeats row by row (the
    ! persistent loop sums in another order)
    rc = fg_set_option(model, FG_OPT_FUSED_DECODE, 0_c_int32_t)
    if (rc /= FG_OK) call stop_rc('fg_set_option', rc)
    call prefill(kv2)
    t0 = now()
    if (ngen > 0) then
      rc = fg_decode_greedy(model, kv2, ids(nprompt:nprompt), ngen, plain, c_null_ptr)
      if (rc /= FG_OK) call stop_rc('fg_decode_greedy', rc)
    end if
    t1 = now()
    ! speculative (spec_bench's run_spec with the lookup drafter)
    call prefill(kv)
    t2 = now()
    rc = fg_decode_spec(model, kv, ids, int(nprompt, c_int32_t), int(ntot, c_int32_t), cfg, st)
    if (rc /= FG_OK) call stop_rc('fg_decode_spec', rc)
    t2 = now() - t2

    open (newunit=u, file=trim(out_file), status='replace', action='write')
    do i = nprompt + 1, ntot
      write (u, '(I0)') ids(i)
    end do
    close (u)
    write (*, '(A,F10.1,A,F10.2)') 'plain : ', 1000*(t1 - t0), ' ms   ', &
        real(ngen, 8)/max(t1 - t0, 1d-9), ' tok/s'
    write (*, '(A,F10.1,A,F10.2)') 'spec  : ', 1000*t2, ' ms   ', real(ngen, 8)/max(t2, 1d-9), ' tok/s'
    write (*, '(A,F8.2,A)') 'speedup: ', (t1 - t0)/max(t2, 1d-9), 'x'
    write (*, '(A,I0,A,F8.2,A,F8.2,A,I0,A,I0)') 'passes=', st%passes, ' tokens/pass=', &
        real(ngen - st%plain, 8)/max(1d0, real(st%passes, 8)), ' mean n_accept=', &
        real(st%accepted, 8)/max(1d0, real(st%passes, 8)), ' plain=', st%plain, &
        ' pauses=', st%pauses
    write (*, '(A,F8.2)') 'mean acceptance rate (nacc/k_eff) = ', &
        real(st%accepted, 8)/max(1d0, real(st%proposed, 8))
    if (ngen == 0) then
      write (*, '(A)') 'EQUIVALENCE ok: spec stream == plain greedy stream'
    else if (all(ids(nprompt+1:ntot) == plain(1:ngen))) then
      write (*, '(A)') 'EQUIVALENCE ok: spec stream == plain greedy stream'
    else
      write (*, '(A)') 'EQUIVALENCE FAILED: spec stream differs from plain greedy'
      stop 1
    end if
    rc = fg_kv_destroy(kv)
    rc = fg_kv_destroy(kv2)
    rc = fg_model_destroy(model)

  contains

    ! a fresh cache holding the prompt minus its last id, in chunks of 64
    subroutine prefill(c)
      type(c_ptr), intent(out) :: c
      rc = fg_kv_create(model, 1_c_int32_t, int(ntot, c_int32_t), c)
      if (rc /= FG_OK) call stop_rc('fg_kv_create', rc)
      srow = 1
      do while (srow <= nprompt - 1)
        tb = min(64, nprompt - srow)
        rc = fg_step_multi(model, c, ids(srow:srow+tb-1), int(tb, c_int32_t), lg, c_null_ptr)
        if (rc /= FG_OK) call stop_rc('fg_step_multi', rc)
        srow = srow + tb
      end do
    end subroutine prefill
  end subroutine run_spec

  subroutine run_sample()
    character(len=512) :: wdir, ids_file, out_file, loop
    integer :: L, D, H, KH, HD, V, ngen, nprompt, ntot, srow, tb, u, i, pwin, nblock, tc
    integer(c_int) :: clen
    integer(c_int32_t) :: rc
    integer(c_int64_t) :: rng
    real(c_float) :: temp, topp, pres, freq, rep, plen
    logical :: bytes
    real(c_float), allocatable :: wte(:), lm(:), c_q(:), c_k(:), c_v(:), c_pr(:), c_fc(:), c_pr2(:)
    real(c_float), allocatable :: cos_b(:), sin_b(:), out1(:), outc(:), ck(:), cv(:)
    integer(c_int), allocatable :: prompt(:), idx(:)
    type(c_ptr) :: model, kv
    type(fg_sample_cfg) :: cfg
    real(8) :: t0, t1

    if (command_argument_count() < 14) call usage()
    wdir = sarg(2); L = iarg(3); D = iarg(4); H = iarg(5); KH = iarg(6); HD = iarg(7); V = iarg(8)
    ids_file = sarg(9); ngen = iarg(10); out_file = sarg(11)
    temp = real(rarg(12), c_float); topp = real(rarg(13), c_float)
    rng = int(iarg(14), c_int64_t)
    pres = 0; freq = 0; rep = 1; pwin = 0; plen = 0; nblock = 0; bytes = .false.; loop = 'host'
    if (command_argument_count() >= 20) then
      pres = real(rarg(15), c_float); freq = real(rarg(16), c_float); rep = real(rarg(17), c_float)
      pwin = iarg(18); plen = real(rarg(19), c_float); nblock = iarg(20)
    end if
    if (command_argument_count() >= 21) bytes = iarg(21) /= 0
    if (command_argument_count() >= 22) loop = sarg(22)

    call load_gpt_weights(trim(wdir), L, D, H, KH, HD, V, wte, lm, c_q, c_k, c_v, c_pr, c_fc, c_pr2)
    call read_ids(trim(ids_file), prompt, nprompt)
    if (nprompt < 1) then
      write (error_unit, '(A)') 'empty prompt'
      stop 1
    end if
    ntot = nprompt + ngen
    allocate (idx(ntot), out1(V), ck(1), cv(1))
    idx(1:nprompt) = prompt(1:nprompt)
    call rope_tables(ntot, HD, cos_b, sin_b)
    clen = 0
    if (nprompt > 1) then
      allocate (outc(max(1, min(64, nprompt - 1))*V))
      srow = 1
      do while (srow <= nprompt - 1)
        tb = min(64, nprompt - srow)
        call gpt_step_multi(idx(srow:srow+tb-1), cos_b((srow-1)*(HD/2)+1:), &
            sin_b((srow-1)*(HD/2)+1:), wte, c_q, c_k, c_v, c_pr, c_fc, c_pr2, lm, &
            ck, cv, clen, ntot, outc, 1, V, D, H, KH, HD, L, tb, 1.0e-5_c_float)
        srow = srow + tb
      end do
    end if
    t0 = now()
    if (trim(loop) == 'device') then
      if (nprompt < 2) then
        write (error_unit, '(A)') 'loop=device needs a prompt of two ids or more'
        stop 2
      end if
      call fgpt_handles(model, kv)
      call set_rope_rows(model, 0, ntot, HD, cos_b, sin_b)
      cfg = fg_sample_cfg(temp, topp, pres, freq, rep, plen, int(pwin, c_int32_t), &
          int(nblock, c_int32_t), merge(1_c_int32_t, 0_c_int32_t, bytes))
      rc = fg_decode_sample(model, kv, idx, int(nprompt, c_int32_t), int(ntot, c_int32_t), cfg, rng)
      if (rc /= FG_OK) call stop_rc('fg_decode_sample', rc)
    else
      do tc = nprompt, ntot - 1
        call gpt_step(idx(tc:tc), cos_b((tc-1)*(HD/2)+1:), sin_b((tc-1)*(HD/2)+1:), &
            wte, c_q, c_k, c_v, c_pr, c_fc, c_pr2, lm, ck, cv, clen, ntot, out1, &
            1, V, D, H, KH, HD, L, 1.0e-5_c_float)
        idx(tc + 1) = sample_next(out1, V, temp, topp, pres, freq, rep, pwin, plen, &
            idx(nprompt+1:), tc - nprompt, nblock, rng, byte_space=bytes) - 1
      end do
    end if
    t1 = now()
    open (newunit=u, file=trim(out_file), status='replace', action='write')
    do i = nprompt + 1, ntot
      write (u, '(I0)') idx(i)
    end do
    close (u)
    write (*, '(A,I0)') 'rng_state=', rng
    write (error_unit, '(A,F10.3,A,F12.1,2A)') 'stats: decode_ms=', 1000*(t1 - t0), &
        ' tok_s=', real(ngen, 8)/max(t1 - t0, 1d-9), ' loop=', trim(loop)
    call fgpt_release()
  end subroutine run_sample

end program fgpt_run
