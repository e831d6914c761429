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
!   selftest cached steps == full forward (src/test/test_kernels.f90:720-779)
!            through the drop-in subroutines on frand-filled weights.
!   spec     greedy speculative decoding as chat_text --spec runs it
!            (src/app/chat_text.f90:293-422: prompt-lookup drafts, one
!            verification pass per round, the sliding-window controller),
!            checked against a plain greedy run on a second cache as
!            src/app/spec_bench.f90 does; prints its summary lines.
!   sample   chat_text's plain loop with sample_next (src/app/chat_text.f90:
!            423-462, src/lib/sample.f90:153-233): loop=host steps through the
!            drop-in gpt_step and sample_next, loop=device is one
!            fg_decode_sample call; the history is the ids generated so far.
!   specbench src/app/spec_bench.f90's truncated-drafter pilot through the
!            drop-in calls: the drafter is the first DL layers of the same
!            stacked weights, each model with its own caller cache; both
!            caches prefilled by gpt_step_multi chunks of 64, a plain greedy
!            run (gpt_step per id, host argmax), then draft-and-verify
!            rounds (K+1 drafter gpt_step calls, one target gpt_step_multi
!            over K+1 rows, accept_prefix, both cache_len rolled back to
!            p-1). Prints spec_bench's summary lines and stops unless the
!            two streams are equal; OUT_FILE gets the plain stream.
!
! Usage:
!   fgpt_run greedy WDIR L D H KH HD V IDS_FILE NGEN OUT_FILE [PCHUNK] [host|device]
!   fgpt_run eval   WDIR L D H KH HD V ROWS_FILE B T OUT_FILE [f16]
!   fgpt_run bpb    WDIR L D H KH HD V ROWS_NPY TOKEN_BYTES [BATCH] [NLL_OUT]
!   fgpt_run selftest
!   fgpt_run spec   WDIR L D H KH HD V IDS_FILE NGEN OUT_FILE [K] [MATCH] [PROBE] [MIN_ACC]
!   fgpt_run specbench WDIR L D H KH HD V IDS_FILE NPRE NGEN OUT_FILE [K] [DL]
!   fgpt_run sample WDIR L D H KH HD V IDS_FILE NGEN OUT_FILE TEMP TOPP SEED
!                   [PRES FREQ REP PWIN PLEN NBLOCK BYTE(0|1) [host|device]]
! Ids files are whitespace-separated 0-based integers. Timing goes to stderr.
program fgpt_run
  use, intrinsic :: iso_c_binding
  use, intrinsic :: iso_fortran_env, only: error_unit, int64
  use fgpt_c
  use fgpt_drop_in_mod
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
  case ('selftest')
    call run_selftest()
  case ('spec')
    call run_spec()
  case ('specbench')
    call run_specbench()
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
    write (error_unit, '(A)') '       fgpt_run selftest'
    write (error_unit, '(A)') '       fgpt_run spec WDIR L D H KH HD V IDS NGEN OUT [K] [MATCH] [PROBE] [MIN_ACC]'
    write (error_unit, '(A)') '       fgpt_run specbench WDIR L D H KH HD V IDS NPRE NGEN OUT [K] [DL]'
    write (error_unit, '(A)') '       fgpt_run sample WDIR L D H KH HD V IDS NGEN OUT TEMP TOPP SEED ' // &
        '[PRES FREQ REP PWIN PLEN NBLOCK BYTE [host|device]]'
    stop 2
  end subroutine usage

  integer function iarg(i)
    integer, intent(in) :: i
    character(len=64) :: s
    integer :: ios
    call get_command_argument(i, s)
    read (s, *, iostat=ios) iarg
    if (ios /= 0) then
      write (error_unit, '(A,I0,2A)') 'bad integer argument ', i, ': ', trim(s)
      stop 2
    end if
  end function iarg

  real(8) function rarg(i)
    integer, intent(in) :: i
    character(len=64) :: s
    integer :: ios
    call get_command_argument(i, s)
    read (s, *, iostat=ios) rarg
    if (ios /= 0) then
      write (error_unit, '(A,I0,2A)') 'bad real argument ', i, ': ', trim(s)
      stop 2
    end if
  end function rarg

  character(len=512) function sarg(i)
    integer, intent(in) :: i
    call get_command_argument(i, sarg)
  end function sarg

  ! Every whitespace-separated integer of the file, in order (any number per
  ! line).
  subroutine read_ids(path, ids, n)
    character(*), intent(in) :: path
    integer(c_int), allocatable, intent(out) :: ids(:)
    integer, intent(out) :: n
    integer :: u, ios, j, nt
    integer(c_int), allocatable :: tmp(:)
    character(len=65536) :: line
    logical :: intok
    allocate (ids(1024))
    n = 0
    open (newunit=u, file=path, status='old', action='read', iostat=ios)
    if (ios /= 0) then
      write (error_unit, '(2A)') 'cannot open ', trim(path)
      stop 1
    end if
    do
      read (u, '(A)', iostat=ios) line
      if (ios /= 0) exit
      nt = 0
      intok = .false.
      do j = 1, len_trim(line)
        if (line(j:j) == ' ' .or. line(j:j) == char(9) .or. line(j:j) == ',') then
          intok = .false.
        else if (.not. intok) then
          intok = .true.
          nt = nt + 1
        end if
      end do
      if (nt == 0) cycle
      do while (n + nt > size(ids))
        allocate (tmp(2*size(ids)))
        tmp(1:size(ids)) = ids
        call move_alloc(tmp, ids)
      end do
      read (line, *, iostat=ios) ids(n+1:n+nt)
      if (ios /= 0) then
        write (error_unit, '(2A)') 'bad ids line in ', trim(path)
        stop 1
      end if
      n = n + nt
    end do
    close (u)
  end subroutine read_ids

  ! chat_text.f90:225-235 / eval_bpb.f90:117-126
  subroutine rope_tables(ntot, hd, cos_b, sin_b)
    integer, intent(in) :: ntot, hd
    real(c_float), allocatable, intent(out) :: cos_b(:), sin_b(:)
    integer :: i, j
    real(c_float) :: theta, ang
    allocate (cos_b(ntot*(hd/2)), sin_b(ntot*(hd/2)))
    do i = 1, ntot
      do j = 1, hd/2
        theta = 10000.0_c_float ** (-2.0_c_float * real(j-1, c_float) / real(hd, c_float))
        ang = real(i-1, c_float) * theta
        cos_b((i-1)*(hd/2)+j) = cos(ang)
        sin_b((i-1)*(hd/2)+j) = sin(ang)
      end do
    end do
  end subroutine rope_tables

  ! RoPE rows [pos0, pos0+n) of the host tables into the engine (the device
  ! loop reads them without a host round trip per step)
  subroutine set_rope_rows(model, pos0, n, hd, cos_b, sin_b)
    type(c_ptr), intent(in) :: model
    integer(c_int), intent(in) :: pos0
    integer, intent(in) :: n, hd
    real(c_float), intent(in) :: cos_b(:), sin_b(:)
    integer(c_int32_t) :: rc
    if (n < 1) return
    rc = fg_set_rope(model, pos0, n, cos_b(pos0*(hd/2)+1:), sin_b(pos0*(hd/2)+1:))
    if (rc /= FG_OK) then
      write (error_unit, '(2A)') 'fg_set_rope: ', fg_error_message()
      stop 1
    end if
  end subroutine set_rope_rows

  real(8) function now()
    integer(int64) :: c, r
    call system_clock(c, r)
    now = real(c, 8) / real(r, 8)
  end function now

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

  subroutine stop_rc(what, rc)
    character(*), intent(in) :: what
    integer(c_int32_t), intent(in) :: rc
    write (error_unit, '(4A,I0,A)') what, ': ', fg_error_message(), ' (rc ', rc, ')'
    stop 1
  end subroutine stop_rc

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

    ! plain greedy on its own cache (spec_bench's run_plain)
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

  ! src/app/spec_bench.f90:132-339 with the drop-in calls underneath
  subroutine run_specbench()
    character(len=512) :: wdir, ids_file, out_file
    integer :: L, D, H, KH, HD, V, npre, ngen, kspec, dl, nmax, d2, nids, i, u
    integer :: clen_t, clen_d, p, npass, naccept_total, ksum, gen_done
    integer, allocatable :: ids(:), prompt(:), seq_plain(:), seq_spec(:), draft(:), targ(:)
    real(c_float), allocatable :: wte(:), lm(:), c_q(:), c_k(:), c_v(:), c_pr(:), c_fc(:), c_pr2(:)
    real(c_float), allocatable :: cos_b(:), sin_b(:), ck_t(:), cv_t(:), ck_d(:), cv_d(:)
    real(c_float), allocatable :: chunk_out(:), row1(:)
    real(8) :: ms_plain, ms_spec, t0

    if (command_argument_count() < 12) call usage()
    wdir = sarg(2); L = iarg(3); D = iarg(4); H = iarg(5); KH = iarg(6); HD = iarg(7); V = iarg(8)
    ids_file = sarg(9); npre = iarg(10); ngen = iarg(11); out_file = sarg(12)
    kspec = 8
    if (command_argument_count() >= 13) kspec = iarg(13)
    dl = 3
    if (command_argument_count() >= 14) dl = iarg(14)
    if (dl < 1 .or. dl > L) then
      write (error_unit, '(A,I0)') 'draft-layers must be in 1..', L
      stop 1
    end if
    if (kspec < 1) then
      write (error_unit, '(A)') 'spec must be >= 1'
      stop 1
    end if
    call read_ids(trim(ids_file), prompt, nids)
    if (nids < npre + 2) then
      write (error_unit, '(A,I0,A,I0)') 'row has ', nids, ' ids, need >= ', npre + 2
      stop 1
    end if
    nmax = npre + ngen + kspec + 4
    d2 = HD / 2
    allocate (ids(nmax + 1))
    ids = 0
    ids(1:npre) = prompt(1:npre)
    call load_gpt_weights(trim(wdir), L, D, H, KH, HD, V, wte, lm, c_q, c_k, c_v, c_pr, c_fc, c_pr2)
    ! the reference's cache shapes: the drop-in keys its device caches by them
    allocate (ck_t(L*nmax*KH*HD), cv_t(L*nmax*KH*HD), ck_d(dl*nmax*KH*HD), cv_d(dl*nmax*KH*HD))
    allocate (chunk_out(max(64, kspec + 2)*V), row1(V))
    allocate (seq_plain(ngen), seq_spec(ngen), draft(kspec), targ(kspec + 1))
    call rope_tables(nmax, HD, cos_b, sin_b)

    write (*, '(A,I0,A,I0,A,I0,A,I0)') 'prompt=', npre, ' gen=', ngen, ' spec K=', kspec, &
        ' drafter layers=', dl
    write (*, '(A,A,A,I0)') 'drafter: ', 'trunc', '  match=', 3

    ! plain greedy: one cached step per token
    clen_t = 0
    clen_d = 0
    call prefill_both()
    t0 = now()
    p = npre
    do i = 1, ngen
      call gpt_step(ids(p:p), cos_b((p-1)*d2+1:), sin_b((p-1)*d2+1:), wte, c_q, c_k, c_v, c_pr, &
          c_fc, c_pr2, lm, ck_t, cv_t, clen_t, nmax, row1, 1, V, D, H, KH, HD, L, 1.0e-5_c_float)
      ids(p + 1) = argmax_i(row1, V) - 1
      seq_plain(i) = ids(p + 1)
      p = p + 1
    end do
    ms_plain = 1000*(now() - t0)

    ! greedy draft-and-verify on the same state
    ids(npre+1:) = 0
    clen_t = 0
    clen_d = 0
    call prefill_both()
    npass = 0
    naccept_total = 0
    ksum = 0
    p = npre
    gen_done = 0
    t0 = now()
    do while (gen_done < ngen)
      call spec_round()
    end do
    ms_spec = 1000*(now() - t0)
    seq_spec(1:ngen) = ids(npre+1:npre+ngen)

    write (*, '(A,F10.1,A,F10.2,A)') 'plain : ', ms_plain, ' ms   ', &
        ngen / max(1.0d-6, ms_plain/1000), ' tok/s'
    write (*, '(A,F10.1,A,F10.2,A)') 'spec  : ', ms_spec, ' ms   ', &
        ngen / max(1.0d-6, ms_spec/1000), ' tok/s'
    write (*, '(A,F8.2,A)') 'speedup: ', ms_plain / max(1.0d-6, ms_spec), 'x'
    write (*, '(A,F8.2,A,F8.2,A,F8.2)') 'passes=', real(npass), ' tokens/pass=', &
        real(ngen)/real(max(1, npass)), ' mean n_accept=', real(naccept_total)/real(max(1, npass))
    write (*, '(A,F8.2)') 'mean acceptance rate (nacc/k_eff) = ', &
        real(naccept_total) / real(max(1, ksum))
    write (*, '(A,F8.2)') 'mean drafts proposed per pass = ', real(ksum) / real(max(1, npass))
    open (newunit=u, file=trim(out_file), status='replace', action='write')
    do i = 1, ngen
      write (u, '(I0)') seq_plain(i)
    end do
    close (u)
    call fgpt_release()
    if (all(seq_plain == seq_spec)) then
      write (*, '(A)') 'EQUIVALENCE ok: spec stream == plain greedy stream'
    else
      write (*, '(A)') 'EQUIVALENCE FAILED: spec stream differs from plain greedy'
      stop 1
    end if

  contains

    integer function argmax_i(x, n)
      integer, intent(in) :: n
      real(c_float), intent(in) :: x(n)
      integer :: t
      argmax_i = 1
      do t = 2, n
        if (x(t) > x(argmax_i)) argmax_i = t
      end do
    end function argmax_i

    ! positions 1..npre-1 into both caches, chunks of 64
    subroutine prefill_both()
      integer :: srow, tb
      srow = 1
      do while (srow <= npre - 1)
        tb = min(64, npre - srow)
        call gpt_step_multi(ids(srow:srow+tb-1), cos_b((srow-1)*d2+1:), sin_b((srow-1)*d2+1:), &
            wte, c_q, c_k, c_v, c_pr, c_fc, c_pr2, lm, ck_t, cv_t, clen_t, nmax, chunk_out, &
            1, V, D, H, KH, HD, L, tb, 1.0e-5_c_float)
        call gpt_step_multi(ids(srow:srow+tb-1), cos_b((srow-1)*d2+1:), sin_b((srow-1)*d2+1:), &
            wte, c_q, c_k, c_v, c_pr, c_fc, c_pr2, lm, ck_d, cv_d, clen_d, nmax, chunk_out, &
            1, V, D, H, KH, HD, dl, tb, 1.0e-5_c_float)
        srow = srow + tb
      end do
    end subroutine prefill_both

    ! one draft-and-verify round; invariant clen_t = clen_d = p-1, ids(p)
    ! the pending token
    subroutine spec_round()
      integer :: inp(kspec + 1), j, na, corr
      call gpt_step(ids(p:p), cos_b((p-1)*d2+1:), sin_b((p-1)*d2+1:), wte, c_q, c_k, c_v, c_pr, &
          c_fc, c_pr2, lm, ck_d, cv_d, clen_d, nmax, row1, 1, V, D, H, KH, HD, dl, 1.0e-5_c_float)
      draft(1) = argmax_i(row1, V) - 1
      do j = 1, kspec - 1
        call gpt_step(draft(j:j), cos_b((p+j-1)*d2+1:), sin_b((p+j-1)*d2+1:), wte, c_q, c_k, &
            c_v, c_pr, c_fc, c_pr2, lm, ck_d, cv_d, clen_d, nmax, row1, 1, V, D, H, KH, HD, dl, &
            1.0e-5_c_float)
        draft(j + 1) = argmax_i(row1, V) - 1
      end do
      ! keeps the drafter cache valid through p+K for the all-accepted case
      call gpt_step(draft(kspec:kspec), cos_b((p+kspec-1)*d2+1:), sin_b((p+kspec-1)*d2+1:), &
          wte, c_q, c_k, c_v, c_pr, c_fc, c_pr2, lm, ck_d, cv_d, clen_d, nmax, row1, 1, V, D, H, &
          KH, HD, dl, 1.0e-5_c_float)
      ksum = ksum + kspec
      inp(1) = ids(p)
      inp(2:kspec+1) = draft(1:kspec)
      call gpt_step_multi(inp, cos_b((p-1)*d2+1:), sin_b((p-1)*d2+1:), wte, c_q, c_k, c_v, &
          c_pr, c_fc, c_pr2, lm, ck_t, cv_t, clen_t, nmax, chunk_out, 1, V, D, H, KH, HD, L, &
          kspec + 1, 1.0e-5_c_float)
      do j = 1, kspec + 1
        targ(j) = argmax_i(chunk_out((j-1)*V+1:j*V), V) - 1
      end do
      call accept_prefix(draft, targ, kspec, na, corr)
      naccept_total = naccept_total + na
      npass = npass + 1
      if (na > 0) ids(p+1:p+na) = draft(1:na)
      ids(p + na + 1) = corr
      p = p + na + 1
      gen_done = p - npre
      ! both caches back to one behind the new pending token
      clen_t = p - 1
      clen_d = p - 1
    end subroutine spec_round
  end subroutine run_specbench

  ! frand of src/test/test_kernels.f90:115-119, explicit 32-bit wrap
  real(c_float) function frand(seed)
    integer, intent(inout) :: seed
    integer(int64) :: t
    t = int(seed, int64) * 1103515245_int64 + 12345_int64
    t = iand(t, int(z'FFFFFFFF', int64))
    if (t >= 2147483648_int64) t = t - 4294967296_int64
    seed = int(mod(t, 2147483647_int64))
    frand = real(mod(seed / 65536, 32768), c_float) / 32768.0_c_float - 0.5_c_float
  end function frand

  subroutine fill(x, scale, seed)
    real(c_float), intent(out) :: x(:)
    real(c_float), intent(in) :: scale
    integer, intent(inout) :: seed
    integer :: i
    do i = 1, size(x)
      ! bf16-exact values: the engine stores weights as bf16
      x(i) = transfer(iand(transfer(frand(seed)*scale, 0), -65536), 0.0_c_float)
    end do
  end subroutine fill

  ! cached steps == full forward, the reference's test_kv_equiv, at dims the
  ! engine supports (head_dim 64, d_model 128)
  subroutine run_selftest()
    integer, parameter :: TC = 6, VV = 128, DD = 128, NH = 2, NKV = 1, HDm = 64, NL = 2
    integer(c_int) :: idx(TC), clen
    real(c_float) :: wte(VV*DD), c_q(NL*NH*HDm*DD), c_k(NL*NKV*HDm*DD), c_v(NL*NKV*HDm*DD)
    real(c_float) :: c_proj(NL*DD*NH*HDm), c_fc(NL*4*DD*DD), c_proj2(NL*DD*4*DD), lm(VV*DD)
    real(c_float) :: out_full(TC*VV), out_steps(TC*VV), out1(VV), ck(1), cv(1)
    real(c_float), allocatable :: cos_b(:), sin_b(:)
    real(c_float) :: err
    integer :: i, t, seed

    seed = 42
    do i = 1, TC
      idx(i) = 1 + mod(i, 7)
    end do
    call fill(wte, 0.1_c_float, seed)
    call fill(c_q, 0.05_c_float, seed)
    call fill(c_k, 0.05_c_float, seed)
    call fill(c_v, 0.05_c_float, seed)
    call fill(c_proj, 0.05_c_float, seed)
    call fill(c_fc, 0.05_c_float, seed)
    call fill(c_proj2, 0.05_c_float, seed)
    call fill(lm, 0.05_c_float, seed)
    call rope_tables(TC, HDm, cos_b, sin_b)
    call gpt_forward(idx, cos_b, sin_b, wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, lm, &
        out_full, 1, TC, VV, DD, NH, NKV, HDm, NL, 1.0e-5_c_float)
    clen = 0
    do t = 1, TC
      call gpt_step(idx(t:t), cos_b((t-1)*(HDm/2)+1:), sin_b((t-1)*(HDm/2)+1:), &
          wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, lm, ck, cv, clen, TC, out1, &
          1, VV, DD, NH, NKV, HDm, NL, 1.0e-5_c_float)
      out_steps((t-1)*VV+1:t*VV) = out1
    end do
    err = maxval(abs(out_full - out_steps)) / maxval(abs(out_full))
    print '(A,ES10.3,A,I0)', 'selftest: cached steps vs forward, max rel err = ', err, &
        '  cache_len=', clen
    call fgpt_release()
    if (clen /= TC .or. .not. (err < 1.0e-5)) then
      print '(A)', 'selftest: FAIL'
      stop 1
    end if
    print '(A)', 'selftest: ok'
  end subroutine run_selftest

end program fgpt_run
