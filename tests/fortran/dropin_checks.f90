! dropin_checks.f90 -- checks of the Fortran drop-in subroutines
! (autoresearch_amd/fortran/fgpt_drop_in.f90) run the way the reference's
! callers run them; test code, built by build() next to this file.
!
!   selftest   cached steps == full forward (src/test/test_kernels.f90:
!              720-779) through gpt_forward / gpt_step on frand weights.
!   specbench  src/app/spec_bench.f90's truncated-drafter pilot: the
!              drafter is the first DL layers of the same stacked weights,
!              each model with its own caller cache; both caches prefilled
!              by gpt_step_multi chunks of 64, a plain greedy run (gpt_step
!              per id, host argmax), then draft-and-verify rounds (K+1
!              drafter gpt_step calls, one target gpt_step_multi over K+1
!              rows, accept_prefix, both cache_len rolled back to p-1).
!              Prints spec_bench's summary lines and stops unless the two
!              streams are equal; OUT_FILE gets the plain stream.
!   posfrac    eval_bpb's --attn blas statistics (src/app/eval_bpb.f90:
!              156-162, src/lib/fortran_attn.f90:247-300): gpt_forward with
!              attn_blas and pos_frac / pos_n over B rows of T ids, called
!              NCALL times into the same accumulators, then once with
!              attn_blas off (the reference leaves them alone then);
!              OUT_FILE gets pos_frac (one per head, %.9e) and pos_n.
!
! Usage:
!   dropin_checks selftest
!   dropin_checks specbench WDIR L D H KH HD V IDS_FILE NPRE NGEN OUT_FILE [K] [DL]
!   dropin_checks posfrac   WDIR L D H KH HD V ROWS_FILE B T NCALL OUT_FILE
program dropin_checks
  use, intrinsic :: iso_c_binding
  use, intrinsic :: iso_fortran_env, only: error_unit, int64
  use fgpt_c
  use fgpt_drop_in_mod
  use fgpt_util
  implicit none

  character(len=512) :: mode

  if (command_argument_count() < 1) call usage()
  call get_command_argument(1, mode)
  select case (trim(mode))
  case ('selftest')
    call run_selftest()
  case ('specbench')
    call run_specbench()
  case ('posfrac')
    call run_posfrac()
  case default
    call usage()
  end select

contains

  subroutine usage()
    write (error_unit, '(A)') 'usage: dropin_checks selftest'
    write (error_unit, '(A)') '       dropin_checks specbench WDIR L D H KH HD V IDS NPRE NGEN OUT [K] [DL]'
    write (error_unit, '(A)') '       dropin_checks posfrac WDIR L D H KH HD V ROWS B T NCALL OUT'
    stop 2
  end subroutine usage

  subroutine run_posfrac()
    character(len=512) :: wdir, rows_file, out_file
    integer :: L, D, H, KH, HD, V, B, T, ncall, n, i, u
    integer(c_int), allocatable :: ids(:)
    real(c_float), allocatable :: wte(:), lm(:), c_q(:), c_k(:), c_v(:), c_pr(:), c_fc(:), c_pr2(:)
    real(c_float), allocatable :: cos_b(:), sin_b(:), outp(:), posf(:)
    integer, allocatable :: posc(:)

    if (command_argument_count() < 13) call usage()
    wdir = sarg(2); L = iarg(3); D = iarg(4); H = iarg(5); KH = iarg(6); HD = iarg(7); V = iarg(8)
    rows_file = sarg(9); B = iarg(10); T = iarg(11); ncall = iarg(12); out_file = sarg(13)
    call read_ids(trim(rows_file), ids, n)
    if (n < B*T) then
      write (error_unit, '(A,I0,A,I0)') 'rows file has ', n, ' ids, need ', B*T
      stop 1
    end if
    call load_gpt_weights(trim(wdir), L, D, H, KH, HD, V, wte, lm, c_q, c_k, c_v, c_pr, c_fc, c_pr2)
    call rope_tables(T, HD, cos_b, sin_b)
    allocate (outp(B*T*V), posf(H), posc(H))
    ! eval_bpb zeroes them once and accumulates over its calls
    posf = 0.0_c_float
    posc = 0
    do i = 1, ncall
      call gpt_forward(ids(1:B*T), cos_b, sin_b, wte, c_q, c_k, c_v, c_pr, c_fc, c_pr2, lm, &
          outp, B, T, V, D, H, KH, HD, L, 1.0e-5_c_float, attn_blas=.true., pos_frac=posf, &
          pos_n=posc)
    end do
    call gpt_forward(ids(1:B*T), cos_b, sin_b, wte, c_q, c_k, c_v, c_pr, c_fc, c_pr2, lm, &
        outp, B, T, V, D, H, KH, HD, L, 1.0e-5_c_float, attn_blas=.false., pos_frac=posf, &
        pos_n=posc)
    open (newunit=u, file=trim(out_file), status='replace', action='write')
    do i = 1, H
      write (u, '(ES17.9E2,1X,I0)') posf(i), posc(i)
    end do
    close (u)
    call fgpt_release()
  end subroutine run_posfrac

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

end program dropin_checks
