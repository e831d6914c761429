! spectest_kats.f90 -- accept_prefix and lookup_draft through the drop-in
! names, on the known answers of src/test/test_kernels.f90:1556-1650 (host
! functions of the engine library: no device is needed). Built and run by
! tests/test_fortran_host.py.
program spectest_kats
  use fgpt_drop_in_mod, only: accept_prefix, lookup_draft
  implicit none
  integer, parameter :: K = 5, NT = 40
  integer :: draft(K), targ(K+1), tg(NT+K+1), buf(NT+K+1), ids(9), d(6)
  integer :: na, corr, p, j, ncomm, npass, ncorr, kk, nfail, nchk

  nfail = 0
  nchk = 0
  draft(1:4) = [1, 2, 3, 4]
  targ(1:5) = [1, 2, 9, 9, 7]
  call accept_prefix(draft, targ, 4, na, corr)
  call chk(na == 2 .and. corr == 9, 'partial match')
  draft(1:3) = [1, 2, 3]
  targ(1:4) = [1, 2, 3, 5]
  call accept_prefix(draft, targ, 3, na, corr)
  call chk(na == 3 .and. corr == 5, 'all match: bonus row')
  draft(1:2) = [1, 2]
  targ(1:3) = [7, 8, 9]
  call accept_prefix(draft, targ, 2, na, corr)
  call chk(na == 0 .and. corr == 7, 'first rejected')
  targ(1) = 4
  call accept_prefix(draft, targ, 0, na, corr)
  call chk(na == 0 .and. corr == 4, 'k=0 is a plain step')
  ! a simulated target stream with a planted draft error every 7th round:
  ! the committed stream must be the target stream
  do j = 1, NT + K + 1
    tg(j) = mod(j*7 + 3, 11)
  end do
  p = 1
  ncomm = 0
  npass = 0
  ncorr = 0
  do while (ncomm < NT .and. p <= NT)
    draft(1:K) = tg(p:p+K-1)
    if (mod(p, 7) == 0) draft(3) = mod(draft(3) + 1, 11)
    targ(1:K+1) = tg(p:p+K)
    call accept_prefix(draft, targ, K, na, corr)
    buf(ncomm+1:ncomm+na) = draft(1:na)
    buf(ncomm+na+1) = corr
    if (na < K) ncorr = ncorr + 1
    ncomm = ncomm + na + 1
    p = p + na + 1
    npass = npass + 1
  end do
  call chk(ncomm >= NT, 'simulation commits the span')
  call chk(all(buf(1:ncomm) == tg(1:ncomm)), 'committed stream == target stream')
  call chk(ncorr > 0, 'reject path exercised')
  ids = [5, 1, 2, 3, 9, 1, 2, 3, 7]
  call lookup_draft(ids, 8, 3, 6, d, kk)
  call chk(kk == 4 .and. all(d(1:4) == [9, 1, 2, 3]), 'continuation capped at known ids')
  call lookup_draft(ids, 8, 3, 2, d, kk)
  call chk(kk == 2 .and. all(d(1:2) == [9, 1]), 'k truncates')
  ids(1:3) = [5, 1, 2]
  call lookup_draft(ids, 3, 5, 4, d, kk)
  call chk(kk == 0, 'm > p-1 is a miss')
  ids(1:6) = [1, 2, 3, 4, 5, 6]
  call lookup_draft(ids, 6, 2, 3, d, kk)
  call chk(kk == 0, 'no earlier occurrence')
  ids(1:6) = [7, 8, 9, 7, 8, 9]
  call lookup_draft(ids, 6, 3, 5, d, kk)
  call chk(kk == 3 .and. all(d(1:3) == [7, 8, 9]), 'match at position 1')
  write (*, '(A,I0,A,I0,A)') 'spectest: ', nchk - nfail, ' of ', nchk, ' checks passed'
  if (nfail > 0) stop 1

contains

  subroutine chk(ok, what)
    logical, intent(in) :: ok
    character(*), intent(in) :: what
    nchk = nchk + 1
    if (.not. ok) then
      nfail = nfail + 1
      write (*, '(2A)') 'FAIL: ', what
    end if
  end subroutine chk
end program spectest_kats
